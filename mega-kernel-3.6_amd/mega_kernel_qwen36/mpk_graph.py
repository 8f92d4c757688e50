"""Decode task graphs and their launch plans.

The reference plans a decode step as a graph of tasks (mega_kernel_qwen36/
mpk_graph.py:37-485): tensors, tasks with dependencies, activation events
(tasks with the same prerequisites share one event), a deterministic
topological order, and a linearized plan whose steps say which tasks run
ahead of time on a fixed worker ("aot") and which are dispatched at run time
("jit").  It never executes a plan.  This module builds the same graphs and
plans -- task ids, kinds, tensors, events and launch steps are an interface
(plans are exchanged as JSON), so they follow the reference -- and
``executor.DecodePlanExecutor`` runs them on the HIP kernels.

A worker here is a compute unit of the GPU: ``WorkerConfig.current_device()``
reads the CU count (256 on an MI355X).  The vision graph is not built: the
vision tower is not part of the decode path.
"""

from __future__ import annotations

import heapq
import json
from dataclasses import dataclass, field, replace
from typing import Any, Callable, Iterable, Mapping, Optional, Sequence

from .config import Qwen36TextConfig, qwen36_27b_config

GridDim = tuple[int, int, int]

# Kinds whose work does not depend on data seen at run time: planned ahead of
# time on a fixed worker (reference mpk_graph.py:236-249).
AOT_KINDS = frozenset({
    "metadata", "embed", "rmsnorm", "linear", "rmsnorm_linear", "linear_residual", "dense_gate_up", "dense_down",
    "vision_patch_embed", "vision_pos_embed", "vision_patch_merger", "argmax",
})
# Kinds whose work depends on run-time data (sequence lengths, routing):
# dispatched just in time (reference mpk_graph.py:250).
JIT_KINDS = frozenset({"paged_attention", "split_kv_attention", "linear_attention", "moe_router",
                       "moe_grouped_experts"})


def _ceil_div(a: int, b: int) -> int:
    return -(-a // b)


def _pow2_sizes(max_batch: int) -> tuple[int, ...]:
    """1, 2, 4, ... below max_batch, then max_batch itself."""
    if max_batch < 1:
        raise ValueError("max_batch must be positive")
    sizes = []
    b = 1
    while b < max_batch:
        sizes.append(b)
        b *= 2
    if not sizes or sizes[-1] != max_batch:
        sizes.append(max_batch)
    return tuple(sizes)


def _grid_for_dim(dim: int, workers: int, tile: int = 64) -> GridDim:
    """One block per `tile` outputs, rounded up to whole waves of workers
    once there are more blocks than workers."""
    blocks = max(1, _ceil_div(dim, tile))
    if workers > 0 and blocks > workers:
        blocks = _ceil_div(blocks, workers) * workers
    return (blocks, 1, 1)


@dataclass(frozen=True)
class TensorSpec:
    name: str
    dims: tuple
    dtype: str = "bf16"
    io_category: str = "cuda_tensor"


@dataclass(frozen=True)
class TaskSpec:
    id: str
    kind: str
    inputs: tuple = ()
    outputs: tuple = ()
    depends_on: tuple = ()
    grid_dim: GridDim = (1, 1, 1)
    block_dim: GridDim = (256, 1, 1)  # four 64-wide waves
    attrs: Mapping[str, Any] = field(default_factory=dict)
    trigger_event: str = ""
    completion_event: str = ""
    launch_mode: str = "aot"
    worker_hint: Optional[int] = None
    scheduler_hint: Optional[int] = None


@dataclass(frozen=True)
class EventSpec:
    id: str
    prerequisites: tuple = ()
    dependents: tuple = ()
    fused_from: tuple = ()


@dataclass(frozen=True)
class WorkerConfig:
    """Workers are compute units; `scheduler_sms` of them (field names as in
    the reference's plans) are set aside for the run-time schedulers, each
    running `scheduler_warps_per_sm` scheduler waves."""

    total_sms: int = 256
    scheduler_sms: int = 4
    scheduler_warps_per_sm: int = 4
    shared_memory_page_kb: int = 32

    @property
    def num_workers(self) -> int:
        return max(1, self.total_sms - self.scheduler_sms)

    @property
    def num_local_schedulers(self) -> int:
        return max(1, self.scheduler_sms * self.scheduler_warps_per_sm)

    @classmethod
    def for_device(cls, total_sms: int, *, scheduler_sms: int = 4) -> "WorkerConfig":
        return cls(total_sms=total_sms, scheduler_sms=min(scheduler_sms, max(1, total_sms - 1)))

    @classmethod
    def current_device(cls) -> "WorkerConfig":
        """CU count of the current GPU (the default config without one)."""
        try:
            import torch

            if torch.cuda.is_available():
                return cls.for_device(torch.cuda.get_device_properties(torch.cuda.current_device())
                                      .multi_processor_count)
        except Exception:  # no GPU runtime: plan for an MI355X
            pass
        return cls()

    current_cuda = current_device  # the reference's name


@dataclass(frozen=True)
class LaunchStep:
    task_id: str
    event_id: str
    launch_mode: str
    worker: Optional[int]
    scheduler: int


@dataclass(frozen=True)
class CompiledPlan:
    graph: "TaskGraph"
    worker_config: WorkerConfig
    launch_steps: tuple
    batch_size: int

    def to_dict(self) -> dict:
        data = self.graph.to_dict()
        wc = self.worker_config
        data["worker_config"] = {
            "total_sms": wc.total_sms,
            "num_workers": wc.num_workers,
            "scheduler_sms": wc.scheduler_sms,
            "num_local_schedulers": wc.num_local_schedulers,
            "shared_memory_page_kb": wc.shared_memory_page_kb,
        }
        data["batch_size"] = self.batch_size
        data["launch_steps"] = [dict(vars(s)) for s in self.launch_steps]
        return data


@dataclass
class TaskGraph:
    name: str
    tensors: dict = field(default_factory=dict)
    tasks: list = field(default_factory=list)
    events: dict = field(default_factory=dict)
    start_event: str = "e_start"

    def add_tensor(self, name: str, dims: Sequence, *, dtype: str = "bf16",
                   io_category: str = "cuda_tensor") -> TensorSpec:
        spec = TensorSpec(name, tuple(dims), dtype, io_category)
        self.tensors[name] = spec
        return spec

    def add_task(self, task_id: str, kind: str, *, inputs: Iterable[str] = (), outputs: Iterable[str] = (),
                 depends_on: Iterable[str] = (), grid_dim: GridDim = (1, 1, 1), block_dim: GridDim = (256, 1, 1),
                 attrs: Optional[Mapping[str, Any]] = None) -> TaskSpec:
        if any(t.id == task_id for t in self.tasks):
            raise ValueError(f"duplicate task id: {task_id}")
        task = TaskSpec(id=task_id, kind=kind, inputs=tuple(inputs), outputs=tuple(outputs),
                        depends_on=tuple(depends_on), grid_dim=grid_dim, block_dim=block_dim,
                        attrs=dict(attrs or {}))
        self.tasks.append(task)
        return task

    def normalize(self) -> "TaskGraph":
        """One activation event per distinct set of prerequisites (tasks that
        wait for the same tasks share it); each task records the event that
        triggers it and its own completion event."""
        event_of: dict = {(): self.start_event}
        members: dict = {self.start_event: []}
        tasks = []
        for t in self.tasks:
            deps = tuple(dict.fromkeys(t.depends_on))  # duplicates dropped, order kept
            ev = event_of.get(deps)
            if ev is None:
                ev = f"e_{len(event_of)}"
                event_of[deps] = ev
                members[ev] = []
            members[ev].append(t.id)
            tasks.append(replace(t, depends_on=deps, trigger_event=ev, completion_event=f"e_done_{t.id}"))
        self.tasks = tasks
        self.events = {
            ev: EventSpec(id=ev, prerequisites=deps, dependents=tuple(members.get(ev, ())),
                          fused_from=tuple(f"e_after_{d}" for d in deps) if len(deps) > 1 else ())
            for deps, ev in event_of.items()
        }
        return self

    event_fusion = normalize

    def topological_tasks(self) -> tuple:
        """Kahn's order, always taking the smallest ready task id (so a plan
        is reproducible); raises on a cycle or a missing dependency."""
        by_id = {t.id: t for t in self.tasks}
        waiting = {t.id: set(t.depends_on) for t in self.tasks}
        users: dict = {}
        for t in self.tasks:
            for d in t.depends_on:
                users.setdefault(d, []).append(t.id)
        ready = [tid for tid, deps in waiting.items() if not deps]
        heapq.heapify(ready)
        order = []
        while ready:
            tid = heapq.heappop(ready)
            order.append(by_id[tid])
            for u in users.get(tid, ()):
                waiting[u].discard(tid)
                if not waiting[u]:
                    heapq.heappush(ready, u)
        if len(order) != len(self.tasks):
            left = sorted(set(by_id) - {t.id for t in order})
            raise ValueError(f"cycle or missing task dependency: {left}")
        return tuple(order)

    def linearize(self, worker_config: Optional[WorkerConfig] = None, *, batch_size: int = 1) -> CompiledPlan:
        wc = worker_config or WorkerConfig.current_device()
        self.normalize()
        steps, planned = [], []
        for ordinal, t in enumerate(self.topological_tasks()):
            if t.kind in JIT_KINDS:
                mode, worker = "jit", None
            elif t.kind in AOT_KINDS or len(t.depends_on) == 1:
                mode, worker = "aot", ordinal % wc.num_workers
            else:
                mode, worker = "jit", None
            sched = ordinal % wc.num_local_schedulers
            planned.append(replace(t, launch_mode=mode, worker_hint=worker, scheduler_hint=sched))
            steps.append(LaunchStep(t.id, t.trigger_event or self.start_event, mode, worker, sched))
        self.tasks = planned
        return CompiledPlan(graph=self, worker_config=wc, launch_steps=tuple(steps), batch_size=batch_size)

    def to_dict(self) -> dict:
        self.normalize()
        return {
            "name": self.name,
            "start_event": self.start_event,
            "tensors": [dict(vars(s)) for s in self.tensors.values()],
            "events": [dict(vars(e)) for e in self.events.values()],
            "tasks": [{**vars(t), "attrs": dict(t.attrs)} for t in self.tasks],
        }

    def to_json(self, *, indent: int = 2) -> str:
        return json.dumps(self.to_dict(), indent=indent, sort_keys=True)


def build_batch_specialized_plans(builder: Callable[[int], TaskGraph], *, max_batch: int,
                                  worker_config: Optional[WorkerConfig] = None) -> dict:
    """One plan per batch size 1, 2, 4, ..., max_batch."""
    return {b: builder(b).linearize(worker_config=worker_config, batch_size=b) for b in _pow2_sizes(max_batch)}


def build_qwen36_decode_tgraph(config: Optional[Qwen36TextConfig] = None, *, batch_size: int = 1,
                               num_layers: Optional[int] = None, include_metadata: bool = True,
                               include_sampling: bool = True,
                               worker_config: Optional[WorkerConfig] = None) -> TaskGraph:
    """The decode step of a Qwen3.6 text model: per layer an input RMSNorm,
    the mixer (qkv projection, paged attention and output projection with
    the residual for full-attention layers; the recurrent linear attention
    with its residual otherwise), the FFN RMSNorm, then the MoE (router,
    grouped experts, down projection with the residual) or the dense SwiGLU
    FFN; then the final norm and, optionally, the LM head and sampling.
    Task ids, kinds and tensors follow the reference (mpk_graph.py:310-485)."""
    cfg = config or qwen36_27b_config()
    wc = worker_config or WorkerConfig.current_device()
    workers = wc.num_workers
    n_layers = cfg.num_hidden_layers if num_layers is None else min(num_layers, cfg.num_hidden_layers)
    B, H = batch_size, cfg.hidden_size
    g = TaskGraph(name=f"{cfg.model_name}:decode:batch{B}")
    g.add_tensor("tokens", (B, "seq"), dtype="int64")
    g.add_tensor("hidden_0", (B, H))
    prev: tuple = ()
    if include_metadata:
        g.add_task("continuous_batching_update", "metadata", inputs=("tokens",), outputs=("decode_metadata",),
                   attrs={"paged_attention": True, "select_power_of_two_tgraph": True})
        g.add_tensor("decode_metadata", (B,), dtype="int32")
        prev = ("continuous_batching_update",)
    g.add_task("embed", "embed", inputs=("tokens",), outputs=("hidden_0",), depends_on=prev,
               attrs={"vocab_size": cfg.vocab_size})
    last = "embed"
    for i in range(n_layers):
        L = f"layer_{i}"
        g.add_tensor(f"{L}_attn_norm_out", (B, H))
        g.add_task(f"{L}_attn_norm", "rmsnorm", inputs=(f"hidden_{i}",), outputs=(f"{L}_attn_norm_out",),
                   depends_on=(last,), grid_dim=(B, 1, 1))
        if cfg.layer_types[i] == "full_attention":
            qh, kvh, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
            qkv_dim = (qh + 2 * kvh) * hd
            g.add_tensor(f"{L}_qkv", (B, qkv_dim))
            g.add_tensor(f"{L}_attn_out", (B, qh * hd))
            g.add_tensor(f"{L}_attn_residual", (B, H))
            g.add_task(f"{L}_qkv_proj", "linear", inputs=(f"{L}_attn_norm_out",), outputs=(f"{L}_qkv",),
                       depends_on=(f"{L}_attn_norm",), grid_dim=_grid_for_dim(qkv_dim, workers),
                       attrs={"projection": "qkv", "head_dim": hd})
            g.add_task(f"{L}_paged_attention", "paged_attention", inputs=(f"{L}_qkv", "decode_metadata"),
                       outputs=(f"{L}_attn_out",), depends_on=(f"{L}_qkv_proj",), grid_dim=(B, kvh, 1),
                       attrs={"causal": True, "kv_heads": kvh, "q_heads": qh})
            g.add_task(f"{L}_attn_out_proj_residual", "linear_residual", inputs=(f"{L}_attn_out", f"hidden_{i}"),
                       outputs=(f"{L}_attn_residual",), depends_on=(f"{L}_paged_attention",),
                       grid_dim=_grid_for_dim(H, workers))
            mixer = f"{L}_attn_out_proj_residual"
        else:
            g.add_tensor(f"{L}_attn_residual", (B, H))
            g.add_task(f"{L}_linear_attention_recurrent", "linear_attention",
                       inputs=(f"{L}_attn_norm_out", f"{L}_linear_state"),
                       outputs=(f"{L}_attn_residual", f"{L}_linear_state_next"), depends_on=(f"{L}_attn_norm",),
                       grid_dim=(B, cfg.linear_num_key_heads, 1),
                       attrs={"key_heads": cfg.linear_num_key_heads, "value_heads": cfg.linear_num_value_heads,
                              "conv_kernel": cfg.linear_conv_kernel_dim})
            mixer = f"{L}_linear_attention_recurrent"
        g.add_tensor(f"{L}_ffn_norm_out", (B, H))
        g.add_task(f"{L}_ffn_norm", "rmsnorm", inputs=(f"{L}_attn_residual",), outputs=(f"{L}_ffn_norm_out",),
                   depends_on=(mixer,), grid_dim=(B, 1, 1))
        g.add_tensor(f"hidden_{i + 1}", (B, H))
        if cfg.is_moe:
            k, E, I = cfg.num_experts_per_tok, cfg.num_experts, cfg.moe_intermediate_size
            g.add_tensor(f"{L}_topk_indices", (B, k), dtype="int64")
            g.add_tensor(f"{L}_topk_weights", (B, k), dtype="float32")
            g.add_tensor(f"{L}_expert_acts", (B, k, I))
            g.add_task(f"{L}_moe_router_topk", "moe_router", inputs=(f"{L}_ffn_norm_out",),
                       outputs=(f"{L}_topk_indices", f"{L}_topk_weights"), depends_on=(f"{L}_ffn_norm",),
                       grid_dim=(B, E, 1), attrs={"experts": E, "top_k": k})
            g.add_task(f"{L}_moe_grouped_experts", "moe_grouped_experts",
                       inputs=(f"{L}_ffn_norm_out", f"{L}_topk_indices", f"{L}_topk_weights"),
                       outputs=(f"{L}_expert_acts",), depends_on=(f"{L}_moe_router_topk",), grid_dim=(B * k, 1, 1),
                       attrs={"intermediate": I, "shared_expert": True})
            g.add_task(f"{L}_moe_down_residual", "linear_residual", inputs=(f"{L}_expert_acts", f"{L}_attn_residual"),
                       outputs=(f"hidden_{i + 1}",), depends_on=(f"{L}_moe_grouped_experts",),
                       grid_dim=_grid_for_dim(H, workers))
            last = f"{L}_moe_down_residual"
        else:
            g.add_tensor(f"{L}_dense_mid", (B, cfg.intermediate_size))
            g.add_task(f"{L}_dense_gate_up", "dense_gate_up", inputs=(f"{L}_ffn_norm_out",),
                       outputs=(f"{L}_dense_mid",), depends_on=(f"{L}_ffn_norm",),
                       grid_dim=_grid_for_dim(2 * cfg.intermediate_size, workers), attrs={"activation": "silu_mul"})
            g.add_task(f"{L}_dense_down_residual", "dense_down", inputs=(f"{L}_dense_mid", f"{L}_attn_residual"),
                       outputs=(f"hidden_{i + 1}",), depends_on=(f"{L}_dense_gate_up",),
                       grid_dim=_grid_for_dim(H, workers))
            last = f"{L}_dense_down_residual"
    g.add_tensor("norm_out", (B, H))
    g.add_task("final_norm", "rmsnorm", inputs=(f"hidden_{n_layers}",), outputs=("norm_out",), depends_on=(last,),
               grid_dim=(B, 1, 1))
    if include_sampling:
        g.add_tensor("logits", (B, cfg.vocab_size))
        g.add_tensor("next_tokens", (B, 1), dtype="int64")
        g.add_task("lm_head", "linear", inputs=("norm_out",), outputs=("logits",), depends_on=("final_norm",),
                   grid_dim=_grid_for_dim(cfg.vocab_size, workers, tile=128))
        g.add_task("argmax_or_sampler", "argmax", inputs=("logits",), outputs=("next_tokens",),
                   depends_on=("lm_head",), grid_dim=(workers, 1, 1))
    return g.normalize()
