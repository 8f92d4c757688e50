"""CPU tests of the boundary: the C ABI library, the Python API's host logic,
error behaviour and configs.  No GPU is touched (the C entry points are only
called with arguments their validation rejects before any HIP call)."""

import ctypes
import pathlib
import re

import pytest
import torch

import mega_kernel_qwen36 as mk
from mega_kernel_qwen36 import _lib

REPO = pathlib.Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "mkq.h"


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mkq_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.library_path()))
    names = header_functions()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), f"{name} declared in include/mkq.h but not exported"


def test_ctypes_signatures_mirror_header():
    assert sorted(_lib.SIGNATURES) == header_functions()


def test_abi_version_and_error_string():
    lib = _lib.load_library()
    assert lib.mkq_abi_version() == 100
    assert isinstance(lib.mkq_last_error(), bytes)


def test_c_abi_rejects_bad_arguments_without_gpu():
    lib = _lib.load_library()
    rc = lib.mkq_dense_ffn_decode(_lib.MKQ_DTYPE_BF16, None, None, None, None, None, None, 0, 16, 16, 1e-6, 1,
                                  None, 0, None)
    assert rc == _lib.MKQ_ERR_INVALID
    assert b"sizes must be positive" in lib.mkq_last_error()
    rc = lib.mkq_moe_decode(_lib.MKQ_DTYPE_BF16, *([None] * 13), 1, 16, 4, 8, 8, 5, 1e-6, 1, None, 0, None)
    assert rc == _lib.MKQ_ERR_INVALID
    assert b"top_k must be in [1, experts]" in lib.mkq_last_error()
    rc = lib.mkq_full_attention_decode(_lib.MKQ_DTYPE_BF16, None, None, None, None, 1, 6, 4, 64, 8, 1.0, None, 0,
                                       None)
    assert rc == _lib.MKQ_ERR_INVALID
    assert b"query_heads must be divisible by kv_heads" in lib.mkq_last_error()
    rc = lib.mkq_full_attention_decode(_lib.MKQ_DTYPE_BF16, None, None, None, None, 1, 4, 4, 512, 8, 1.0, None, 0,
                                       None)
    assert b"head_dim > 256" in lib.mkq_last_error()
    rc = lib.mkq_gated_delta_decode(_lib.MKQ_DTYPE_BF16, *([None] * 8), 1, 3, 4, 8, 8, None)
    assert rc == _lib.MKQ_ERR_INVALID
    assert b"multiple of k_heads" in lib.mkq_last_error()


def test_noalloc_moe_entry_validates_on_the_host_without_gpu():
    """The no-allocation MoE entry point rejects bad arguments, and shapes
    whose workspace exceeds its static scratch array, before any HIP call."""
    lib = _lib.load_library()
    rc = lib.mkq_moe_decode_noalloc(_lib.MKQ_DTYPE_BF16, *([None] * 13), 1, 16, 4, 8, 8, 5, 1e-6, 1, None)
    assert rc == _lib.MKQ_ERR_INVALID
    assert b"top_k must be in [1, experts]" in lib.mkq_last_error()
    rc = lib.mkq_moe_decode_noalloc(_lib.MKQ_DTYPE_BF16, *([None] * 13), 1, 2048, 256, 512, 512, 8, 1e-6, 1, None)
    assert rc == _lib.MKQ_ERR_INVALID
    assert b"moe_decode_noalloc: null tensor pointer" in lib.mkq_last_error()
    # experts 1024, top-64, intermediate 1024: a 33 MB workspace, beyond the 8 MiB array
    need = lib.mkq_moe_decode_workspace_bytes(1, 2048, 1024, 1024, 1024, 64)
    assert need > 8 << 20
    dummy = [256] * 13  # never dereferenced: the size check comes first
    rc = lib.mkq_moe_decode_noalloc(_lib.MKQ_DTYPE_BF16, *dummy, 1, 2048, 1024, 1024, 1024, 64, 1e-6, 1, None)
    assert rc == _lib.MKQ_ERR_UNSUPPORTED
    msg = lib.mkq_last_error()
    assert b"needs %d bytes of scratch" % need in msg and b"holds %d" % (8 << 20) in msg
    # config 2 fits
    assert lib.mkq_moe_decode_workspace_bytes(8, 2048, 256, 512, 512, 8) <= 8 << 20


def test_rms_norm_gemv_entry_validates_on_the_host_without_gpu():
    lib = _lib.load_library()
    rc = lib.mkq_rms_norm_gemv(_lib.MKQ_DTYPE_BF16, None, None, 1e-6, None, None, 0, 16, 16, None)
    assert rc == _lib.MKQ_ERR_INVALID and b"sizes must be positive" in lib.mkq_last_error()
    rc = lib.mkq_rms_norm_gemv(_lib.MKQ_DTYPE_BF16, 256, None, 1e-6, 256, 256, 1, 16, 16, None)
    assert rc == _lib.MKQ_ERR_INVALID and b"rms_norm_gemv: null tensor pointer" in lib.mkq_last_error()
    rc = lib.mkq_rms_norm_gemv(_lib.MKQ_DTYPE_BF16, 256, 256, -1.0, 256, 256, 1, 16, 16, None)
    assert rc == _lib.MKQ_ERR_INVALID and b"eps must be non-negative" in lib.mkq_last_error()


def test_decode_layer_projection_shape_errors_before_device_work():
    """A qkv_proj / in_proj whose row count does not split into the heads is a
    ValueError; on CPU tensors the HIP path refuses before any device work."""
    x = torch.zeros(1, 32, dtype=torch.bfloat16)
    att = mk.FullAttentionInputs(q=None, k_cache=torch.zeros(1, 4, 2, 8), v_cache=torch.zeros(1, 4, 2, 8),
                                 qkv_proj=torch.zeros(30, 32), input_norm=torch.ones(32))
    with pytest.raises(RuntimeError, match="decode_layer input projection"):
        mk.decode_layer(3, x, None, full_attention=att)


def test_rope_entry_rejects_unsupported_rotary_dims_without_gpu():
    """The in-kernel RoPE entry point validates on the host and returns
    MKQ_ERR_UNSUPPORTED for rotary dims it cannot rotate in the kernel; the
    buffers are host memory and are never touched."""
    lib = _lib.load_library()
    b, hq, hkv, d, t = 1, 4, 2, 64, 8
    nbytes = lib.mkq_full_attention_decode_workspace_bytes(b, hq, hkv, d, t)
    raw = ctypes.create_string_buffer(nbytes + 512)
    ws = (ctypes.addressof(raw) + 255) // 256 * 256
    buf = ctypes.create_string_buffer(4096 + 16)
    p16 = (ctypes.addressof(buf) + 15) // 16 * 16
    for rot in (24, 8, 128):
        rc = lib.mkq_full_attention_decode_rope(_lib.MKQ_DTYPE_BF16, p16, p16, p16, p16, b, hq, hkv, d, t, 1.0, p16,
                                                rot, ws, nbytes, None)
        assert rc == _lib.MKQ_ERR_UNSUPPORTED, rot
        assert b"rotary_dim" in lib.mkq_last_error()
    rc = lib.mkq_full_attention_decode_rope(_lib.MKQ_DTYPE_F32, p16, p16, p16, p16, b, hq, hkv, d, t, 1.0, p16, 32,
                                            ws, nbytes, None)
    assert rc == _lib.MKQ_ERR_UNSUPPORTED
    rc = lib.mkq_full_attention_decode_rope(_lib.MKQ_DTYPE_BF16, p16, p16, p16, p16, b, hq, hkv, d, t, 1.0, None, 32,
                                            ws, nbytes, None)
    assert rc == _lib.MKQ_ERR_INVALID
    assert b"null cos/sin pointer" in lib.mkq_last_error()


def test_append_entry_validates_on_the_host_without_gpu():
    """mkq_full_attention_decode_append rejects what it cannot do before any
    launch: a missing k_new/v_new or a capacity below seq_len (INVALID), and
    FP32 or a head_dim that is not a multiple of 8 (UNSUPPORTED, nothing
    written).  The buffers are host memory and are never touched."""
    lib = _lib.load_library()
    b, hq, hkv, d, t, cap = 1, 4, 2, 64, 8, 16
    nbytes = lib.mkq_full_attention_decode_workspace_bytes(b, hq, hkv, d, t)
    raw = ctypes.create_string_buffer(nbytes + 512)
    ws = (ctypes.addressof(raw) + 255) // 256 * 256
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) // 16 * 16
    call = lib.mkq_full_attention_decode_append
    assert call(_lib.MKQ_DTYPE_BF16, p, None, p, p, p, p, b, hq, hkv, d, t, cap, 1.0, None, 0, ws, nbytes,
                None) == _lib.MKQ_ERR_INVALID
    assert call(_lib.MKQ_DTYPE_BF16, p, p, p, p, p, p, b, hq, hkv, d, t, t - 1, 1.0, None, 0, ws, nbytes,
                None) == _lib.MKQ_ERR_INVALID
    assert b"capacity" in lib.mkq_last_error()
    assert call(_lib.MKQ_DTYPE_F32, p, p, p, p, p, p, b, hq, hkv, d, t, cap, 1.0, None, 0, ws, nbytes,
                None) == _lib.MKQ_ERR_UNSUPPORTED
    assert call(_lib.MKQ_DTYPE_BF16, p, p, p, p, p, p, b, hq, hkv, 20, t, cap, 1.0, None, 0, ws, nbytes,
                None) == _lib.MKQ_ERR_UNSUPPORTED
    assert b"append" in lib.mkq_last_error()


def test_append_inputs_validated_before_any_device_work():
    """The Python KV append checks its arguments first: both of k_new/v_new,
    and a cache_seqlen that leaves a row for the new token."""
    q = torch.zeros(1, 4, 64)
    kc = torch.zeros(1, 8, 2, 64)
    kn = torch.zeros(1, 2, 64)
    with pytest.raises(ValueError, match="together"):
        mk.full_attention_decode(mk.FullAttentionInputs(q, kc, kc.clone(), k_new=kn))
    with pytest.raises(ValueError, match="room"):
        mk.full_attention_decode(mk.FullAttentionInputs(q, kc, kc.clone(), k_new=kn, v_new=kn, cache_seqlen=8))


def test_gemv_add_rejects_null_pointers_without_gpu():
    """mkq_gemv_add needs the residual and both outputs; the checks run on the
    host before any launch, so host buffers are never touched."""
    lib = _lib.load_library()
    buf = ctypes.create_string_buffer(256)
    p = ctypes.addressof(buf)
    for args in ((p, p, None, p, p), (p, p, p, p, None), (p, p, p, None, p)):
        rc = lib.mkq_gemv_add(_lib.MKQ_DTYPE_BF16, *args, 1, 8, 8, None)
        assert rc == _lib.MKQ_ERR_INVALID
        assert b"null tensor pointer" in lib.mkq_last_error()
    rc = lib.mkq_gemv_add(_lib.MKQ_DTYPE_BF16, p, p, p, p, p, 0, 8, 8, None)
    assert rc == _lib.MKQ_ERR_INVALID


def test_workspace_sizes():
    lib = _lib.load_library()
    # act [batch, intermediate] FP32 plus the batched path's fragments, partials and counters
    assert lib.mkq_dense_ffn_decode_workspace_bytes(2, 5120, 17408) >= 2 * 17408 * 4 + 17408 // 32 * 1024
    assert (lib.mkq_dense_ffn_decode_workspace_bytes(8, 5120, 17408)
            - lib.mkq_dense_ffn_decode_workspace_bytes(2, 5120, 17408)) == 6 * 17408 * 4
    assert lib.mkq_moe_decode_workspace_bytes(1, 2048, 256, 512, 512, 8) > 8 * 8 * 512 * 4
    assert lib.mkq_full_attention_decode_workspace_bytes(1, 24, 4, 256, 32768) >= 24 * 32768 * 4


# ---------------------------------------------------------------------------
# Python API host logic (reference ops.py behaviour)
# ---------------------------------------------------------------------------

def _tiny_moe():
    g = torch.Generator().manual_seed(0)
    r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    return r(2, 8), mk.MoeWeights(r(8), r(4, 8), r(4, 6, 8), r(4, 6, 8), r(4, 8, 6), r(6, 8), r(6, 8), r(8, 6))


def test_backend_validation_messages():
    x, w = _tiny_moe()
    with pytest.raises(ValueError, match="backend must be one of: auto, persistent, grouped, reference"):
        mk.moe_decode(x, w, backend="nope")
    dw = mk.DenseFfnWeights(torch.ones(8), torch.ones(4, 8), torch.ones(4, 8), torch.ones(8, 4))
    with pytest.raises(ValueError, match="backend must be one of: auto, torch, triton, reference"):
        mk.dense_ffn_decode(x, dw, backend="nope")


def test_hip_backends_fail_loudly_on_cpu_tensors():
    x, w = _tiny_moe()
    with pytest.raises(RuntimeError, match="GPU|HIP extension"):
        mk.moe_decode(x, w, top_k=2)
    with pytest.raises(RuntimeError, match="GPU|HIP extension"):
        mk.moe_decode(x, w, top_k=2, backend="persistent")
    with pytest.raises(RuntimeError, match="test infrastructure"):
        mk.moe_decode(x, w, top_k=2, backend="reference")
    inp = mk.FullAttentionInputs(q=torch.randn(1, 4, 8), k_cache=torch.randn(1, 3, 2, 8), v_cache=torch.randn(1, 3, 2, 8))
    with pytest.raises(RuntimeError, match="GPU|HIP extension"):
        mk.full_attention_decode(inp)
    bad = mk.FullAttentionInputs(q=torch.randn(1, 3, 8), k_cache=torch.randn(1, 3, 2, 8), v_cache=torch.randn(1, 3, 2, 8))
    with pytest.raises(ValueError, match="query_heads must be divisible by kv_heads"):
        mk.full_attention_decode(bad)


def test_grouped_torch_backend_runs_on_cpu_and_agrees_with_oracle():
    import oracle

    x, w = _tiny_moe()
    out, idx, rw = mk.moe_decode(x, w, top_k=2, backend="grouped")
    ref, ref_idx, ref_w = oracle.moe_decode(*(t.numpy() for t in (x, *w.__dict__.values())), top_k=2)
    assert idx.tolist() == ref_idx.tolist()
    torch.testing.assert_close(out, torch.from_numpy(ref), atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(rw, torch.from_numpy(ref_w))


def test_decode_layer_dispatch_errors():
    x, w = _tiny_moe()
    with pytest.raises(ValueError, match="full_attention inputs are required"):
        mk.decode_layer(3, x, w)
    with pytest.raises(ValueError, match="linear_attention inputs are required"):
        mk.decode_layer(0, x, w)
    with pytest.raises(ValueError, match="unsupported layer_type"):
        mk.decode_layer(0, x, w, layer_type="conv")
    lin = mk.LinearAttentionInputs(q=torch.randn(2, 2, 4), k=torch.randn(2, 2, 4), v=torch.randn(2, 2, 4),
                                   state=torch.zeros(2, 2, 4, 4))
    with pytest.raises(RuntimeError):  # CPU tensors never fall back to a CPU path
        mk.decode_layer(0, x, w, linear_attention=lin)


def test_gated_weights_dataclass_keeps_reference_fields():
    x, w = _tiny_moe()
    gw = mk.GatedMoeWeights(*w.__dict__.values(), shared_expert_gate=torch.zeros(8))
    assert isinstance(gw, mk.MoeWeights)
    assert list(mk.MoeWeights.__dataclass_fields__) == [
        "norm_weight", "router_weight", "expert_gate", "expert_up", "expert_down", "shared_gate", "shared_up",
        "shared_down"]
    assert len(w.__dict__) == 8  # rebuilt by MoeWeights(*w.__dict__.values()) in the reference tests


def test_configs_match_published_dims():
    c = mk.qwen36_35b_a3b_config()
    assert (c.hidden_size, c.num_experts, c.num_experts_per_tok, c.moe_intermediate_size,
            c.shared_expert_intermediate_size) == (2048, 256, 8, 512, 512)
    assert (c.linear_num_key_heads, c.linear_num_value_heads, c.linear_key_head_dim, c.head_dim) == (16, 32, 128, 256)
    d = mk.qwen36_27b_config()
    assert (d.hidden_size, d.intermediate_size, d.num_attention_heads, d.num_key_value_heads) == (5120, 17408, 24, 4)
    assert [mk.qwen36_layer_type(i) for i in range(8)] == ["linear_attention"] * 3 + ["full_attention"] + \
        ["linear_attention"] * 3 + ["full_attention"]
    assert c.rotary_dim == 64


def test_paged_entry_validates_on_the_host_without_gpu():
    """mkq_full_attention_decode_paged checks its layout before any launch:
    a null table, a block size that is not a multiple of 16 or too few blocks
    for seq_len (INVALID), FP32 (UNSUPPORTED).  Host buffers, never touched."""
    lib = _lib.load_library()
    b, hq, hkv, d, t = 1, 4, 2, 64, 40
    nbytes = lib.mkq_full_attention_decode_workspace_bytes(b, hq, hkv, d, t)
    raw = ctypes.create_string_buffer(nbytes + 512)
    ws = (ctypes.addressof(raw) + 255) // 256 * 256
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) // 16 * 16
    call = lib.mkq_full_attention_decode_paged
    assert call(_lib.MKQ_DTYPE_BF16, p, p, p, None, p, b, hq, hkv, d, t, 16, 3, 8, 1.0, ws, nbytes,
                None) == _lib.MKQ_ERR_INVALID
    assert call(_lib.MKQ_DTYPE_BF16, p, p, p, p, p, b, hq, hkv, d, t, 24, 3, 8, 1.0, ws, nbytes,
                None) == _lib.MKQ_ERR_INVALID
    assert b"block_size" in lib.mkq_last_error()
    assert call(_lib.MKQ_DTYPE_BF16, p, p, p, p, p, b, hq, hkv, d, t, 16, 2, 8, 1.0, ws, nbytes,
                None) == _lib.MKQ_ERR_INVALID
    assert call(_lib.MKQ_DTYPE_F32, p, p, p, p, p, b, hq, hkv, d, t, 16, 3, 8, 1.0, ws, nbytes,
                None) == _lib.MKQ_ERR_UNSUPPORTED


def test_linear_step_entry_validates_on_the_host_without_gpu():
    """mkq_linear_attention_step sizes its workspace from the shapes and
    rejects a short or misaligned workspace and a key_dim above 256 before
    any launch."""
    lib = _lib.load_library()
    need = lib.mkq_linear_attention_step_workspace_bytes(_lib.MKQ_DTYPE_BF16, 2, 16, 32, 128, 128)
    # two fixed arrays of 16384 arrival counts, then FP32 output rows [2, 32, 128]
    assert need == 2 * 16384 * 4 + 2 * 32 * 128 * 4
    assert lib.mkq_linear_attention_step_workspace_bytes(99, 2, 16, 32, 128, 128) == 0
    raw = ctypes.create_string_buffer(need + 512)
    ws = (ctypes.addressof(raw) + 255) // 256 * 256
    buf = ctypes.create_string_buffer(256)
    p = ctypes.addressof(buf)
    call = lib.mkq_linear_attention_step
    args = [p, p, p, None, 3, p, p, p, p, p, p, 2, 16, 32, 128, 128, 0.1, 1e-6]
    assert call(_lib.MKQ_DTYPE_BF16, *args, ws, need - 1, None) == _lib.MKQ_ERR_INVALID
    assert b"workspace" in lib.mkq_last_error()
    assert call(_lib.MKQ_DTYPE_BF16, *args, ws + 16, need, None) == _lib.MKQ_ERR_INVALID
    bad = list(args)
    bad[14] = 512  # key_dim
    assert call(_lib.MKQ_DTYPE_BF16, *bad, ws, need, None) == _lib.MKQ_ERR_UNSUPPORTED
    bad = list(args)
    bad[11] = 600  # batch * v_heads above the 16384 arrival counts
    assert call(_lib.MKQ_DTYPE_BF16, *bad, ws, need, None) == _lib.MKQ_ERR_UNSUPPORTED
    assert b"v_heads" in lib.mkq_last_error()
    bad = list(args)
    bad[4] = 8  # conv_state_len: width 9 > 8 taps
    assert call(_lib.MKQ_DTYPE_BF16, *bad, ws, need, None) == _lib.MKQ_ERR_INVALID
    assert b"conv_state_len" in lib.mkq_last_error()


def test_paged_append_entry_rejects_missing_rows_without_gpu():
    lib = _lib.load_library()
    b, hq, hkv, d, t = 1, 4, 2, 64, 40
    nbytes = lib.mkq_full_attention_decode_workspace_bytes(b, hq, hkv, d, t)
    raw = ctypes.create_string_buffer(nbytes + 512)
    ws = (ctypes.addressof(raw) + 255) // 256 * 256
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) // 16 * 16
    call = lib.mkq_full_attention_decode_paged_append
    assert call(_lib.MKQ_DTYPE_BF16, p, None, p, p, p, p, p, b, hq, hkv, d, t, 16, 3, 8, 1.0, ws, nbytes,
                None) == _lib.MKQ_ERR_INVALID
    assert call(_lib.MKQ_DTYPE_F32, p, p, p, p, p, p, p, b, hq, hkv, d, t, 16, 3, 8, 1.0, ws, nbytes,
                None) == _lib.MKQ_ERR_UNSUPPORTED


def test_paged_append_rope_entry_validates_on_the_host_without_gpu():
    """mkq_full_attention_decode_paged_append_rope rejects missing tensors and
    a non-positive rotary_dim before any launch."""
    lib = _lib.load_library()
    b, hq, hkv, d, t = 1, 4, 2, 64, 40
    nbytes = lib.mkq_full_attention_decode_workspace_bytes(b, hq, hkv, d, t)
    raw = ctypes.create_string_buffer(nbytes + 512)
    ws = (ctypes.addressof(raw) + 255) // 256 * 256
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) // 16 * 16
    call = lib.mkq_full_attention_decode_paged_append_rope
    assert call(_lib.MKQ_DTYPE_BF16, p, p, p, p, p, p, p, b, hq, hkv, d, t, 16, 3, 8, 1.0, None, 16, ws, nbytes,
                None) == _lib.MKQ_ERR_INVALID
    assert call(_lib.MKQ_DTYPE_BF16, p, None, p, p, p, p, p, b, hq, hkv, d, t, 16, 3, 8, 1.0, p, 16, ws, nbytes,
                None) == _lib.MKQ_ERR_INVALID
    assert call(_lib.MKQ_DTYPE_BF16, p, p, p, p, p, p, p, b, hq, hkv, d, t, 16, 3, 8, 1.0, p, 0, ws, nbytes,
                None) == _lib.MKQ_ERR_INVALID
    assert b"rotary_dim" in lib.mkq_last_error()
    assert call(_lib.MKQ_DTYPE_BF16, p, p, p, p, p, p, p, b, hq, hkv, d, t, 24, 3, 8, 1.0, p, 16, ws, nbytes,
                None) == _lib.MKQ_ERR_INVALID  # block_size not a multiple of 16


def test_paged_rope_entry_validates_on_the_host_without_gpu():
    """mkq_full_attention_decode_paged_rope checks its arguments before any
    launch: a null table or cos/sin and a non-positive rotary_dim or a block
    size that is not a multiple of 16 (INVALID); FP32 and a rotary_dim that is
    not a power of two in [16, head_dim] (UNSUPPORTED).  Host buffers, never
    touched."""
    lib = _lib.load_library()
    b, hq, hkv, d, t = 1, 4, 2, 64, 40
    nbytes = lib.mkq_full_attention_decode_workspace_bytes(b, hq, hkv, d, t)
    raw = ctypes.create_string_buffer(nbytes + 512)
    ws = (ctypes.addressof(raw) + 255) // 256 * 256
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) // 16 * 16
    call = lib.mkq_full_attention_decode_paged_rope

    def run(dtype=_lib.MKQ_DTYPE_BF16, table=p, cs=p, block_size=16, rot=32):
        return call(dtype, p, p, p, table, p, b, hq, hkv, d, t, block_size, 3, 8, 1.0, cs, rot, ws, nbytes, None)

    assert run(table=None) == _lib.MKQ_ERR_INVALID
    assert run(cs=None) == _lib.MKQ_ERR_INVALID
    assert run(rot=0) == _lib.MKQ_ERR_INVALID
    assert b"rotary_dim" in lib.mkq_last_error()
    assert run(block_size=24) == _lib.MKQ_ERR_INVALID
    assert run(dtype=_lib.MKQ_DTYPE_F32) == _lib.MKQ_ERR_UNSUPPORTED
    for rot in (8, 48, 128):  # below 16, not a power of two, above head_dim
        assert run(rot=rot) == _lib.MKQ_ERR_UNSUPPORTED
        assert b"rotary_dim" in lib.mkq_last_error()


def test_new_python_entry_points_validate_arguments_before_device_work():
    """The paged-KV, conv-update and q/k-norm options reject bad arguments
    with ValueError before touching a device (CPU tensors here)."""
    q = torch.zeros(2, 4, 64)
    pool = torch.zeros(10, 16, 2, 64)
    with pytest.raises(ValueError, match="block_table"):
        mk.full_attention_decode(mk.FullAttentionInputs(q, pool, pool.clone(),
                                                        block_table=torch.zeros(3, 4, dtype=torch.int32)))
    with pytest.raises(ValueError, match="seq_len"):
        mk.full_attention_decode(mk.FullAttentionInputs(q, pool, pool.clone(),
                                                        block_table=torch.zeros(2, 4, dtype=torch.int32),
                                                        seq_len=65))
    with pytest.raises(ValueError, match="together"):
        mk.full_attention_decode(mk.FullAttentionInputs(q, pool, pool.clone(),
                                                        block_table=torch.zeros(2, 4, dtype=torch.int32),
                                                        k_new=torch.zeros(2, 2, 64)))
    with pytest.raises(ValueError, match="activation"):
        mk.causal_conv1d_update(torch.zeros(1, 8), torch.zeros(1, 8, 3), torch.zeros(8, 4), activation="gelu")
    lin = mk.LinearAttentionInputs(q=torch.zeros(1, 2, 8), k=torch.zeros(1, 2, 8), v=torch.zeros(1, 2, 8),
                                   state=torch.zeros(1, 2, 8, 8), qk_l2norm=True)
    with pytest.raises(ValueError, match="qk_l2norm"):
        mk.linear_attention_decode(lin)
