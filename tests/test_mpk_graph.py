"""CPU tests of the decode planner (reference mpk_graph.py's behaviour, as
its tests/test_mpk_graph.py checks it) and of how the executor compiles a
plan into launches; no GPU is touched."""

import json

import pytest
import torch

import mega_kernel_qwen36 as mk


def test_decode_tgraph_contains_events_and_launch_modes():
    graph = mk.build_qwen36_decode_tgraph(mk.qwen36_27b_config(), batch_size=2, num_layers=4,
                                          worker_config=mk.WorkerConfig.for_device(132))
    plan = graph.linearize(worker_config=mk.WorkerConfig.for_device(132), batch_size=2)
    kinds = {task.kind for task in plan.graph.tasks}
    assert {"paged_attention", "linear_attention", "dense_gate_up"} <= kinds
    assert any(step.launch_mode == "jit" for step in plan.launch_steps)
    assert any(step.launch_mode == "aot" for step in plan.launch_steps)
    assert plan.worker_config.num_workers == 128
    assert plan.worker_config.num_local_schedulers == 16


def test_moe_tgraph_has_router_and_grouped_experts():
    graph = mk.build_qwen36_decode_tgraph(mk.qwen36_35b_a3b_config(), batch_size=1, num_layers=1,
                                          include_sampling=False, worker_config=mk.WorkerConfig.for_device(132))
    kinds = [task.kind for task in graph.tasks]
    assert "moe_router" in kinds and "moe_grouped_experts" in kinds
    assert "lm_head" not in [t.id for t in graph.tasks]


def test_batch_specialized_plans_use_powers_of_two():
    plans = mk.build_batch_specialized_plans(
        lambda b: mk.build_qwen36_decode_tgraph(mk.qwen36_27b_config(), batch_size=b, num_layers=1,
                                                worker_config=mk.WorkerConfig.for_device(132)),
        max_batch=8, worker_config=mk.WorkerConfig.for_device(132))
    assert tuple(plans) == (1, 2, 4, 8)
    assert all(p.batch_size == b for b, p in plans.items())
    assert tuple(mk.build_batch_specialized_plans(
        lambda b: mk.build_qwen36_decode_tgraph(num_layers=1), max_batch=6,
        worker_config=mk.WorkerConfig()).keys()) == (1, 2, 4, 6)


def test_plan_json_export_and_event_fusion():
    """Tasks with the same prerequisites share one activation event; a task
    waiting for two tasks gets an event fused from their completions; the
    plan round-trips through JSON; launch order is topological."""
    g = mk.TaskGraph(name="toy")
    g.add_task("a", "rmsnorm")
    g.add_task("b", "linear", depends_on=("a",))
    g.add_task("c", "linear", depends_on=("a",))
    g.add_task("d", "linear_residual", depends_on=("b", "c", "b"))
    plan = g.linearize(worker_config=mk.WorkerConfig.for_device(8), batch_size=1)
    ev = {t.id: t.trigger_event for t in plan.graph.tasks}
    assert ev["a"] == "e_start" and ev["b"] == ev["c"] != ev["d"]
    assert plan.graph.events[ev["d"]].prerequisites == ("b", "c")
    assert plan.graph.events[ev["d"]].fused_from == ("e_after_b", "e_after_c")
    assert [s.task_id for s in plan.launch_steps] == ["a", "b", "c", "d"]
    assert [s.launch_mode for s in plan.launch_steps] == ["aot", "aot", "aot", "aot"]
    data = json.loads(json.dumps(plan.to_dict()))
    assert data["batch_size"] == 1 and data["worker_config"]["num_workers"] == 4
    assert [t["id"] for t in data["tasks"]] == ["a", "b", "c", "d"]
    with pytest.raises(ValueError, match="duplicate task id"):
        g.add_task("a", "rmsnorm")
    g2 = mk.TaskGraph(name="cycle")
    g2.add_task("x", "linear", depends_on=("y",))
    g2.add_task("y", "linear", depends_on=("x",))
    with pytest.raises(ValueError, match="cycle or missing task dependency"):
        g2.linearize(worker_config=mk.WorkerConfig())


def test_decode_plan_launch_modes_follow_task_kinds():
    plan = mk.build_qwen36_decode_tgraph(mk.qwen36_35b_a3b_config(), num_layers=4,
                                         worker_config=mk.WorkerConfig()).linearize(worker_config=mk.WorkerConfig())
    kind = {t.id: t.kind for t in plan.graph.tasks}
    for s in plan.launch_steps:
        if kind[s.task_id] in ("paged_attention", "linear_attention", "moe_router", "moe_grouped_experts"):
            assert s.launch_mode == "jit" and s.worker is None
        else:
            assert s.launch_mode == "aot" and 0 <= s.worker < mk.WorkerConfig().num_workers
    assert mk.WorkerConfig().num_workers == 252  # 256 CUs, 4 for the schedulers


def _cpu_layer(kind, ffn):
    z = torch.zeros
    fa = mk.FullAttentionInputs(q=None, k_cache=z(1, 8, 2, 64), v_cache=z(1, 8, 2, 64), qkv_proj=z(8 * 64, 512),
                                out_proj=z(512, 4 * 64)) if kind == "full" else None
    la = mk.LinearAttentionInputs(q=None, k=None, v=None, state=z(1, 4, 64, 64), g=z(1, 4), beta=z(1, 4),
                                  in_proj=z(512, 512), out_proj=z(512, 256)) if kind == "linear" else None
    moe = mk.MoeWeights(*(z(1) for _ in range(8))) if ffn == "moe" else None
    dense = mk.DenseFfnWeights(*(z(1) for _ in range(4))) if ffn == "dense" else None
    return mk.DecodeLayerWeights(input_norm=z(512), full_attention=fa, linear_attention=la, moe=moe, dense_ffn=dense)


def test_executor_compiles_a_plan_into_fused_launches():
    cfg = mk.Qwen36TextConfig(hidden_size=512, num_hidden_layers=4)
    plan = mk.build_qwen36_decode_tgraph(cfg, num_layers=4, include_metadata=False, include_sampling=False,
                                         worker_config=mk.WorkerConfig()).linearize(worker_config=mk.WorkerConfig())
    layers = [_cpu_layer("linear", "moe")] * 3 + [_cpu_layer("full", "moe")]
    ex = mk.DecodePlanExecutor(plan, layers)
    assert ex.launch_groups() == ((0, "linear_attention"), (0, "moe"), (1, "linear_attention"), (1, "moe"),
                                  (2, "linear_attention"), (2, "moe"), (3, "attn_norm"), (3, "paged_attention"),
                                  (3, "attn_out_proj_residual"), (3, "moe"))
    assert ex.not_executed == ("final_norm",)
    with pytest.raises(ValueError, match="weights for 2 layers"):
        mk.DecodePlanExecutor(plan, layers[:2])
    with pytest.raises(ValueError, match="full_attention part but its weights were not given"):
        mk.DecodePlanExecutor(plan, [_cpu_layer("linear", "moe")] * 4)
    with pytest.raises(ValueError, match="dense part"):
        dense_plan = mk.build_qwen36_decode_tgraph(mk.qwen36_27b_config(), num_layers=1, include_metadata=False,
                                                   include_sampling=False, worker_config=mk.WorkerConfig())
        mk.DecodePlanExecutor(dense_plan.linearize(worker_config=mk.WorkerConfig()), [_cpu_layer("linear", "moe")])
    with pytest.raises(RuntimeError, match="capture"):
        ex.replay()
