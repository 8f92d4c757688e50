"""GPU: a linearized decode plan (the planner's 35B-A3B decode graph, four
layers: three linear-attention layers and one full-attention layer, each with
the config-2 MoE) run by DecodePlanExecutor on the HIP kernels, against the
same layers chained through decode_layer (bit for bit: the same fused
launches), and the whole plan captured into one HIP graph and replayed
(bit for bit with the eager run, several replays with eager work between)."""

import dataclasses

import pytest
import torch

import mega_kernel_qwen36 as mk
from tests.inputs import make_gated_delta, make_moe

pytestmark = pytest.mark.gpu


def _rand(g, *shape, scale=0.02, shift=0.0):
    return (torch.randn(*shape, generator=g) * scale + shift).to("cuda", torch.bfloat16)


def _layers(cfg, g, moe):
    H = cfg.hidden_size
    layers = []
    for i in range(4):
        norm = _rand(g, H, shift=1.0)
        if cfg.layer_types[i] == "full_attention":
            qh, kvh, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
            fa = mk.FullAttentionInputs(
                q=None, k_cache=_rand(g, 1, 1024, kvh, hd, scale=1.0), v_cache=_rand(g, 1, 1024, kvh, hd, scale=1.0),
                scale=hd ** -0.5, out_proj=_rand(g, H, qh * hd), qkv_proj=_rand(g, (qh + 2 * kvh) * hd, H),
                cache_seqlen=900)
            layers.append(mk.DecodeLayerWeights(input_norm=norm, full_attention=fa, moe=moe))
        else:
            lin = make_gated_delta(batch=1, seed=800 + i)
            hk, hv, dk, dv = 16, 32, 128, 128
            lin = dataclasses.replace(lin, q=None, k=None, v=None, qk_l2norm=True,
                                      in_proj=_rand(g, 2 * hk * dk + hv * dv, H), out_proj=_rand(g, H, hv * dv))
            layers.append(mk.DecodeLayerWeights(input_norm=norm, linear_attention=lin, moe=moe))
    return layers


def _chained(layers, x, k):
    for i, w in enumerate(layers):
        fa = dataclasses.replace(w.full_attention, input_norm=w.input_norm) if w.full_attention else None
        la = dataclasses.replace(w.linear_attention, input_norm=w.input_norm) if w.linear_attention else None
        x = mk.decode_layer(i, x, w.moe, full_attention=fa, linear_attention=la, top_k=k).hidden
    return x


def test_executor_runs_a_decode_plan():
    cfg = mk.qwen36_35b_a3b_config()
    plan = mk.build_qwen36_decode_tgraph(cfg, batch_size=1, num_layers=4, include_metadata=False,
                                         include_sampling=False).linearize(batch_size=1)
    x, moe, k = make_moe(batch=1, seed=801)
    g = torch.Generator().manual_seed(802)
    layers = _layers(cfg, g, moe)
    cache0 = layers[3].full_attention.k_cache.clone(), layers[3].full_attention.v_cache.clone()
    ex = mk.DecodePlanExecutor(plan, layers, top_k=k)
    assert [grp for _, grp in ex.launch_groups()].count("moe") == 4
    print("executor: eager run", flush=True)
    res = ex.run(x)
    got_cache = layers[3].full_attention.k_cache.clone(), layers[3].full_attention.v_cache.clone()
    # the same layers through decode_layer, on a fresh copy of the cache
    layers[3].full_attention.k_cache.copy_(cache0[0])
    layers[3].full_attention.v_cache.copy_(cache0[1])
    want = _chained(layers, x, k)
    torch.cuda.synchronize()
    assert torch.equal(res.hidden, want)
    assert torch.equal(got_cache[0], layers[3].full_attention.k_cache)
    assert torch.equal(got_cache[1], layers[3].full_attention.v_cache)
    assert not torch.equal(got_cache[0][:, 900], cache0[0][:, 900])  # the new token was appended
    assert all(res.router_indices[i] is not None for i in range(4))
    assert all(res.linear_states[i] is not None for i in range(3)) and res.linear_states[3] is None
    assert res.not_executed == ("final_norm",)

    print("executor: graph capture and replays", flush=True)
    ex.capture(x)
    for rep in range(3):
        out = ex.replay(x)
        torch.cuda.synchronize()
        assert torch.equal(out.hidden, want), f"replay {rep}"
        assert torch.equal(out.router_indices[0], res.router_indices[0])
        _ = ex.run(x)  # eager work between replays
        torch.cuda.synchronize()
    # per decode step: eager launches vs one graph replay (warm)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = {}
    for name, fn in (("eager", lambda: ex.run(x)), ("graph", lambda: ex.replay())):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(20):
            fn()
        e1.record()
        torch.cuda.synchronize()
        times[name] = e0.elapsed_time(e1) * 1e3 / 20
    print(f"4-layer decode step: eager {times['eager']:.1f} us, graph replay {times['graph']:.1f} us", flush=True)
