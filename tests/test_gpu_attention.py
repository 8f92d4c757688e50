"""GPU parity: GQA full-attention decode (split-K flash-decode on MFMA) vs the oracle.

Tolerance (task): bf16 outputs atol 1e-2, rtol 1e-2.
"""

import math

import numpy as np
import pytest
import torch

import mega_kernel_qwen36 as mk
import oracle
from mega_kernel_qwen36 import _lib
from tests.inputs import assert_close_out, make_attention, np32

pytestmark = pytest.mark.gpu


def _ref(inp):
    return oracle.full_attention_decode(np32(inp.q), np32(inp.k_cache), np32(inp.v_cache), scale=inp.scale)


@pytest.mark.parametrize("seq_len", [1, 128, 4096])
def test_attention_reference_test_shape(seq_len):
    # test_cuda_ops.py:79-90 shape: B 2, Hq 4, Hkv 2, D 32, values * 0.1
    inp = make_attention(batch=2, q_heads=4, kv_heads=2, head_dim=32, seq_len=seq_len, seed=17, scale=0.1)
    out = mk.full_attention_decode(inp)
    assert out.shape == inp.q.shape and out.dtype == inp.q.dtype
    assert_close_out(out, _ref(inp))


@pytest.mark.parametrize("seq_len", [4096, 32768])
def test_attention_config4(seq_len):
    """Config 4: B 1, 24 q heads, 4 kv heads, D 256, contiguous bf16 KV."""
    inp = make_attention(seq_len=seq_len)
    assert_close_out(mk.full_attention_decode(inp), _ref(inp))


def test_attention_config4_128k():
    inp = make_attention(seq_len=131072)
    assert_close_out(mk.full_attention_decode(inp), _ref(inp))


@pytest.mark.parametrize("shape", [
    (1, 24, 4, 256, 1000),   # ragged tail
    (3, 6, 6, 128, 77),      # MHA (group 1)
    (1, 32, 1, 64, 300),     # group 32 -> two head groups
    (2, 8, 2, 40, 50),       # head_dim 40: 8-multiple, partial MFMA step
    (1, 4, 2, 20, 33),       # head_dim 20: generic path
    (1, 12, 2, 96, 4500),    # head_dim 96 on the 128-wide kernel, several chunks
    (2, 40, 2, 128, 2049),   # group 20 -> head groups of 16 and 4, batch 2
    (1, 8, 8, 256, 16),      # exactly one tile
    (1, 24, 4, 256, 65),     # one token past a workgroup pass
])
def test_attention_odd_shapes(shape):
    b, hq, hkv, d, t = shape
    inp = make_attention(batch=b, q_heads=hq, kv_heads=hkv, head_dim=d, seq_len=t, seed=sum(shape))
    assert_close_out(mk.full_attention_decode(inp), _ref(inp))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_attention_other_dtypes(dtype):
    inp = make_attention(batch=1, q_heads=12, kv_heads=2, head_dim=128, seq_len=2000, seed=5, dtype=dtype)
    out = mk.full_attention_decode(inp)
    assert out.dtype == dtype
    assert_close_out(out, _ref(inp))


def test_attention_known_answers():
    # T = 1 => out = v ; constant keys => out = mean(V)
    inp = make_attention(batch=1, q_heads=6, kv_heads=1, head_dim=256, seq_len=1, seed=8)
    out = mk.full_attention_decode(inp)
    expect = np32(inp.v_cache)[:, 0, 0][:, None, :].repeat(6, axis=1)
    assert_close_out(out, expect)
    inp = make_attention(batch=1, q_heads=6, kv_heads=1, head_dim=256, seq_len=513, seed=9)
    k_const = inp.k_cache[:, :1].expand_as(inp.k_cache).contiguous()
    out = mk.full_attention_decode(mk.FullAttentionInputs(q=inp.q, k_cache=k_const, v_cache=inp.v_cache))
    expect = np32(inp.v_cache).mean(axis=1)[:, 0][:, None, :].repeat(6, axis=1)
    assert_close_out(out, expect)


def test_attention_default_scale_and_rope():
    inp = make_attention(batch=1, q_heads=8, kv_heads=2, head_dim=64, seq_len=200, seed=10)
    cos = torch.cos(torch.linspace(0, 3, 32)).repeat(2)[None].expand(200, 64)[:, :32].contiguous()
    sin = torch.sin(torch.linspace(0, 3, 32)).repeat(2)[None].expand(200, 64)[:, :32].contiguous()
    full = mk.FullAttentionInputs(q=inp.q, k_cache=inp.k_cache, v_cache=inp.v_cache, cos=cos[:1], sin=sin[:1],
                                  rotary_dim=32)
    out = mk.full_attention_decode(full)
    qn, kn = oracle.apply_partial_rope(np32(inp.q), np32(inp.k_cache), cos[:1].numpy(), sin[:1].numpy(), 32)
    # the API rounds the rotated q/k back to bf16 before the kernel, as the reference does
    qn, kn = oracle.bf16_round(qn), oracle.bf16_round(kn)
    ref = oracle.full_attention_decode(qn, kn, np32(inp.v_cache), scale=1.0 / math.sqrt(64))
    assert_close_out(out, ref)


def test_attention_deterministic():
    inp = make_attention(batch=1, seq_len=8192, seed=12)
    a = mk.full_attention_decode(inp)
    b = mk.full_attention_decode(inp)
    assert torch.equal(a, b)


def _capi_attention(inp, ws):
    """One call of mkq_full_attention_decode through the C ABI on a caller-owned workspace."""
    lib = _lib.load_library()
    b, hq, d = inp.q.shape
    t, hkv = inp.k_cache.shape[1], inp.k_cache.shape[2]
    out = torch.empty_like(inp.q)
    dtype = {torch.bfloat16: _lib.MKQ_DTYPE_BF16, torch.float16: _lib.MKQ_DTYPE_F16}[inp.q.dtype]
    rc = lib.mkq_full_attention_decode(dtype, inp.q.data_ptr(), inp.k_cache.data_ptr(), inp.v_cache.data_ptr(),
                                       out.data_ptr(), b, hq, hkv, d, t, inp.scale, ws.data_ptr(), ws.numel(),
                                       torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.MKQ_OK, lib.mkq_last_error()
    return out


def test_attention_workspace_reuse_across_paths():
    """One zero-filled workspace, calls of several shapes in turn through the C
    ABI: the split-K kernels (one workgroup per CU at D = 256, two at 128,
    several at 40) and the generic kernel (head_dim 20) share it, and every
    output matches the oracle."""
    lib = _lib.load_library()
    shapes = [(1, 24, 4, 256, 32768), (1, 4, 2, 20, 33), (2, 8, 2, 40, 50), (1, 24, 4, 256, 32768),
              (1, 12, 2, 96, 4500), (1, 24, 4, 256, 1000), (1, 24, 4, 256, 32768)]
    nbytes = max(lib.mkq_full_attention_decode_workspace_bytes(b, hq, hkv, d, t) for b, hq, hkv, d, t in shapes)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    inputs = {}
    for i, key in enumerate(shapes):
        b, hq, hkv, d, t = key
        if key not in inputs:
            inputs[key] = make_attention(batch=b, q_heads=hq, kv_heads=hkv, head_dim=d, seq_len=t, seed=200 + i)
        inp = inputs[key]
        out = _capi_attention(inp, ws)
        torch.cuda.synchronize()
        assert_close_out(out, _ref(inp))


def test_attention_graph_replay():
    """A captured config-4 call (chunk and merge kernels) replays
    bit-identically to the eager call; eager calls of two shapes on the same
    stream, which share the capture's workspace, run between the replays."""
    inp = make_attention(seq_len=32768, seed=21)
    eager = mk.full_attention_decode(inp)
    other = make_attention(batch=1, q_heads=8, kv_heads=2, head_dim=128, seq_len=3000, seed=22)
    other_ref = mk.full_attention_decode(other)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mk.full_attention_decode(inp)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        res = mk.full_attention_decode(inp)
    for _ in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(res, eager)
        with torch.cuda.stream(s):
            mid = mk.full_attention_decode(inp)
            mid2 = mk.full_attention_decode(other)
        torch.cuda.synchronize()
        assert torch.equal(mid, eager)
        assert torch.equal(mid2, other_ref)


def _rope_inputs(shape, rot, seed, dtype=torch.bfloat16):
    b, hq, hkv, d, t = shape
    inp = make_attention(batch=b, q_heads=hq, kv_heads=hkv, head_dim=d, seq_len=t, seed=seed, dtype=dtype)
    g = torch.Generator().manual_seed(seed + 1)
    ang = torch.rand(rot, generator=g) * 6.0
    cos, sin = torch.cos(ang)[None], torch.sin(ang)[None]  # one vector for every token, as the reference broadcasts
    return inp, cos, sin


@pytest.mark.parametrize("shape,rot,dtype", [
    ((1, 24, 4, 256, 4096), 64, torch.bfloat16),
    ((2, 8, 2, 128, 300), 32, torch.bfloat16),
    ((1, 8, 8, 64, 77), 64, torch.bfloat16),       # rotary_dim == head_dim
    ((1, 12, 2, 128, 2000), 16, torch.float16),
    ((1, 24, 4, 256, 65), 128, torch.bfloat16),
])
def test_attention_rope_in_kernel_equals_rotated_cache(shape, rot, dtype):
    """Keys rotated inside the kernel give exactly the output of the plain
    kernel on a cache rotated beforehand (the reference's order,
    reference.py:91-114 then attention_decode.cu), and match the oracle."""
    inp, cos, sin = _rope_inputs(shape, rot, seed=300 + sum(shape) + rot, dtype=dtype)
    fused = mk.full_attention_decode(mk.FullAttentionInputs(q=inp.q, k_cache=inp.k_cache, v_cache=inp.v_cache,
                                                            cos=cos, sin=sin, rotary_dim=rot))
    qr, kr = mk.ops.apply_partial_rope(inp.q, inp.k_cache, cos, sin, rot)
    plain = mk.full_attention_decode(mk.FullAttentionInputs(q=qr, k_cache=kr, v_cache=inp.v_cache))
    assert torch.equal(fused, plain)
    qn, kn = oracle.apply_partial_rope(np32(inp.q), np32(inp.k_cache), cos.numpy(), sin.numpy(), rot)
    qn, kn = oracle.bf16_round(qn), oracle.bf16_round(kn)
    if dtype == torch.bfloat16:
        assert_close_out(fused, oracle.full_attention_decode(qn, kn, np32(inp.v_cache),
                                                             scale=1.0 / math.sqrt(shape[3])))


def test_attention_rope_fallback_rotates_the_cache():
    """A rotary_dim the kernel does not rotate (24) still follows the
    reference: the cache is rotated first, then the plain kernel runs."""
    inp, cos, sin = _rope_inputs((1, 8, 2, 64, 200), 24, seed=401)
    out = mk.full_attention_decode(mk.FullAttentionInputs(q=inp.q, k_cache=inp.k_cache, v_cache=inp.v_cache,
                                                          cos=cos, sin=sin, rotary_dim=24))
    qn, kn = oracle.apply_partial_rope(np32(inp.q), np32(inp.k_cache), cos.numpy(), sin.numpy(), 24)
    qn, kn = oracle.bf16_round(qn), oracle.bf16_round(kn)
    assert_close_out(out, oracle.full_attention_decode(qn, kn, np32(inp.v_cache), scale=1.0 / math.sqrt(64)))


def test_attention_rope_cos_changed_in_place():
    """The device (cos, sin) vector built for the kernel is reused only while
    the same cos/sin tensors are unchanged: an in-place update is seen."""
    inp, cos, sin = _rope_inputs((1, 8, 2, 128, 500), 64, seed=501)
    cos, sin = cos.cuda(), sin.cuda()
    full = mk.FullAttentionInputs(q=inp.q, k_cache=inp.k_cache, v_cache=inp.v_cache, cos=cos, sin=sin, rotary_dim=64)
    first = mk.full_attention_decode(full)
    cos.mul_(-0.5)
    sin.add_(0.25)
    second = mk.full_attention_decode(full)
    qr, kr = mk.ops.apply_partial_rope(inp.q, inp.k_cache, cos, sin, 64)
    plain = mk.full_attention_decode(mk.FullAttentionInputs(q=qr, k_cache=kr, v_cache=inp.v_cache))
    assert torch.equal(second, plain)
    assert not torch.equal(first, second)


def _append_case(b, hq, hkv, d, cap, dtype, seed):
    """q, the new token's k/v and caches of `cap` rows filled with stale values
    everywhere (including the row the new token goes to)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, d, generator=g).to("cuda", dtype)
    k_new = torch.randn(b, hkv, d, generator=g).to("cuda", dtype)
    v_new = torch.randn(b, hkv, d, generator=g).to("cuda", dtype)
    k_cache = torch.randn(b, cap, hkv, d, generator=g).to("cuda", dtype)
    v_cache = torch.randn(b, cap, hkv, d, generator=g).to("cuda", dtype)
    return q, k_new, v_new, k_cache, v_cache


@pytest.mark.parametrize("b,hq,hkv,d,seq,cap,dtype,rot", [
    (1, 24, 4, 256, 32768, 32768, torch.bfloat16, 0),   # config 4, the cache's last row
    (1, 24, 4, 256, 32768, 33000, torch.bfloat16, 64),  # preallocated cache, RoPE in the kernel
    (2, 8, 2, 128, 3001, 4096, torch.float16, 0),       # batch stride = capacity, not seq_len
    (1, 32, 1, 64, 1, 16, torch.bfloat16, 32),          # the new token alone; two head groups
    (3, 40, 2, 128, 700, 1024, torch.bfloat16, 0),      # group 20: two head groups share the row
    (2, 16, 4, 256, 4097, 5000, torch.float16, 128),    # new token first in its tile
])
def test_attention_append_in_kernel_equals_written_cache(b, hq, hkv, d, seq, cap, dtype, rot):
    """KV append inside the attention kernel: the output is bit-identical to
    writing the new row with torch first and attending over the first seq_len
    tokens with the plain (or RoPE) path, and afterwards the caches equal the
    torch-written ones everywhere (the new row written, every other row
    untouched)."""
    q, k_new, v_new, k_cache, v_cache = _append_case(b, hq, hkv, d, cap, dtype, 400 + seq)
    cos = sin = None
    if rot:
        ang = torch.rand(rot, generator=torch.Generator().manual_seed(seq)) * 6.0
        cos, sin = torch.cos(ang)[None], torch.sin(ang)[None]
    k_ref, v_ref = k_cache.clone(), v_cache.clone()
    k_ref[:, seq - 1] = k_new
    v_ref[:, seq - 1] = v_new
    want = mk.full_attention_decode(mk.FullAttentionInputs(
        q, k_ref[:, :seq].contiguous(), v_ref[:, :seq].contiguous(), cos=cos, sin=sin, rotary_dim=rot or 64))
    got = mk.full_attention_decode(mk.FullAttentionInputs(
        q, k_cache, v_cache, cos=cos, sin=sin, rotary_dim=rot or 64, k_new=k_new, v_new=v_new,
        cache_seqlen=seq - 1))
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(k_cache, k_ref)
    assert torch.equal(v_cache, v_ref)
    if rot == 0 and seq <= 4096:
        inp = mk.FullAttentionInputs(q, k_ref[:, :seq].contiguous(), v_ref[:, :seq].contiguous(),
                                     scale=1.0 / math.sqrt(d))
        assert_close_out(got, _ref(inp))


def test_attention_append_through_c_abi_then_next_step():
    """Two decode steps through mkq_full_attention_decode_append on one
    preallocated cache: each step's output matches the oracle on the cache as
    written so far, and the second step reads the row the first one wrote."""
    lib = _lib.load_library()
    b, hq, hkv, d, cap, t0 = 1, 12, 2, 128, 2048, 1500
    q, k_new, v_new, k_cache, v_cache = _append_case(b, hq, hkv, d, cap, torch.bfloat16, 77)
    nbytes = lib.mkq_full_attention_decode_workspace_bytes(b, hq, hkv, d, t0 + 2)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    for step in range(2):
        seq = t0 + 1 + step
        kn = k_new * (step + 1)
        vn = v_new - step
        expect_k, expect_v = k_cache.clone(), v_cache.clone()
        expect_k[:, seq - 1] = kn
        expect_v[:, seq - 1] = vn
        out = torch.empty_like(q)
        rc = lib.mkq_full_attention_decode_append(_lib.MKQ_DTYPE_BF16, q.data_ptr(), kn.data_ptr(), vn.data_ptr(),
                                                  k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(), b, hq, hkv,
                                                  d, seq, cap, 1.0 / math.sqrt(d), None, 0, ws.data_ptr(), nbytes,
                                                  stream)
        assert rc == _lib.MKQ_OK, lib.mkq_last_error()
        torch.cuda.synchronize()
        assert torch.equal(k_cache, expect_k) and torch.equal(v_cache, expect_v)
        inp = mk.FullAttentionInputs(q, k_cache[:, :seq].contiguous(), v_cache[:, :seq].contiguous(),
                                     scale=1.0 / math.sqrt(d))
        assert_close_out(out, _ref(inp))


@pytest.mark.parametrize("d,dtype,rot", [(20, torch.bfloat16, 0), (64, torch.float32, 0), (128, torch.bfloat16, 24)])
def test_attention_append_fallback_writes_then_attends(d, dtype, rot):
    """Shapes the kernel cannot append in place (generic head_dim, FP32, a
    rotary_dim it cannot rotate) write the rows with torch and take the other
    paths; the result and the caches are the same as doing that by hand."""
    b, hq, hkv, seq, cap = 2, 8, 2, 90, 128
    q, k_new, v_new, k_cache, v_cache = _append_case(b, hq, hkv, d, cap, dtype, 500 + d)
    cos = sin = None
    if rot:
        ang = torch.rand(rot, generator=torch.Generator().manual_seed(5)) * 6.0
        cos, sin = torch.cos(ang)[None], torch.sin(ang)[None]
    k_ref, v_ref = k_cache.clone(), v_cache.clone()
    k_ref[:, seq - 1] = k_new
    v_ref[:, seq - 1] = v_new
    want = mk.full_attention_decode(mk.FullAttentionInputs(
        q, k_ref[:, :seq].contiguous(), v_ref[:, :seq].contiguous(), cos=cos, sin=sin, rotary_dim=rot or 64))
    got = mk.full_attention_decode(mk.FullAttentionInputs(
        q, k_cache, v_cache, cos=cos, sin=sin, rotary_dim=rot or 64, k_new=k_new, v_new=v_new, cache_seqlen=seq - 1))
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(k_cache, k_ref) and torch.equal(v_cache, v_ref)


def _paged_case(inp, bs, seed, bad_block=None):
    """Scatter a contiguous cache into a shuffled block pool (padding rows and
    unused blocks hold garbage); returns (pool_k, pool_v, table, expected
    contiguous k/v).  With bad_block=(row, j) that table entry is set outside
    the pool, and the expected cache has zeros there."""
    b, t, hkv, d = inp.k_cache.shape
    nb = (t + bs - 1) // bs
    g = torch.Generator().manual_seed(seed)
    num_blocks = b * nb + 5
    perm = torch.randperm(num_blocks, generator=g)[: b * nb].reshape(b, nb)
    pad = nb * bs - t
    pool_k = torch.randn(num_blocks, bs, hkv, d, generator=g).to("cuda", inp.k_cache.dtype)
    pool_v = torch.randn(num_blocks, bs, hkv, d, generator=g).to("cuda", inp.k_cache.dtype)
    garbage = torch.randn(b, pad, hkv, d, generator=g).to("cuda", inp.k_cache.dtype)
    kp = torch.cat([inp.k_cache, garbage], 1).reshape(b, nb, bs, hkv, d)
    vp = torch.cat([inp.v_cache, garbage], 1).reshape(b, nb, bs, hkv, d)
    for r in range(b):
        pool_k[perm[r].cuda()] = kp[r]
        pool_v[perm[r].cuda()] = vp[r]
    table = torch.full((b, nb + 1), 1 << 30, dtype=torch.int32)
    table[:, :nb] = perm.to(torch.int32)
    k_want, v_want = inp.k_cache.clone(), inp.v_cache.clone()
    if bad_block is not None:
        r, j = bad_block
        table[r, j] = -7
        k_want[r, j * bs:(j + 1) * bs] = 0
        v_want[r, j * bs:(j + 1) * bs] = 0
    return pool_k, pool_v, table.cuda(), k_want, v_want


@pytest.mark.parametrize("b,hq,hkv,d,t,bs,dtype", [
    (1, 24, 4, 256, 32768, 16, torch.bfloat16),   # config 4 in 16-token blocks
    (1, 24, 4, 256, 4096, 256, torch.bfloat16),
    (3, 8, 2, 128, 3001, 64, torch.float16),      # ragged last block
    (2, 40, 2, 128, 700, 32, torch.bfloat16),     # group 20: two head groups
    (1, 4, 4, 64, 1, 16, torch.bfloat16),         # one token
])
def test_attention_paged_equals_contiguous(b, hq, hkv, d, t, bs, dtype):
    """The paged kernel over a shuffled block pool is bit-identical to the
    contiguous kernel over the same tokens; rows past seq_len and unused
    blocks (garbage) are never read."""
    inp = make_attention(batch=b, q_heads=hq, kv_heads=hkv, head_dim=d, seq_len=t, seed=600 + t, dtype=dtype)
    pk, pv, table, _, _ = _paged_case(inp, bs, 601 + t)
    got = mk.full_attention_decode(mk.FullAttentionInputs(inp.q, pk, pv, scale=inp.scale, block_table=table,
                                                          seq_len=t))
    want = mk.full_attention_decode(inp)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    if t <= 4096:
        assert_close_out(got, _ref(inp))


def test_attention_paged_block_outside_pool_reads_zeros():
    """A table entry outside [0, num_blocks) reads as zeros instead of
    faulting: the result equals the contiguous kernel with those rows zeroed."""
    inp = make_attention(batch=2, q_heads=8, kv_heads=2, head_dim=128, seq_len=1000, seed=610)
    pk, pv, table, kz, vz = _paged_case(inp, 64, 611, bad_block=(1, 3))
    got = mk.full_attention_decode(mk.FullAttentionInputs(inp.q, pk, pv, scale=inp.scale, block_table=table,
                                                          seq_len=1000))
    want = mk.full_attention_decode(mk.FullAttentionInputs(inp.q, kz, vz, scale=inp.scale))
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("d,bs,dtype", [(128, 8, torch.bfloat16), (20, 16, torch.bfloat16), (64, 16, torch.float32)])
def test_attention_paged_fallback_gathers(d, bs, dtype):
    """Block sizes or head dims the kernel does not read in place are gathered
    into a contiguous cache first; the result equals the contiguous path."""
    inp = make_attention(batch=2, q_heads=4, kv_heads=2, head_dim=d, seq_len=77, seed=620 + d, dtype=dtype)
    pk, pv, table, _, _ = _paged_case(inp, bs, 621)
    got = mk.full_attention_decode(mk.FullAttentionInputs(inp.q, pk, pv, scale=inp.scale, block_table=table,
                                                          seq_len=77))
    want = mk.full_attention_decode(inp)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("b,hq,hkv,d,t,bs,dtype", [
    (1, 24, 4, 256, 32768, 16, torch.bfloat16),   # config 4, 16-token blocks
    (3, 8, 2, 128, 3001, 64, torch.float16),      # ragged last block
    (2, 40, 2, 128, 1, 16, torch.bfloat16),       # the first token of a fresh block; group 20
    (2, 4, 2, 128, 77, 8, torch.bfloat16),        # block size the kernel does not take: written first
])
def test_attention_paged_append_equals_write_then_attend(b, hq, hkv, d, t, bs, dtype):
    """KV append into a paged pool: the output and both pools are
    bit-identical to writing the new row into its block with torch and then
    attending over the pool; no other row changes."""
    inp = make_attention(batch=b, q_heads=hq, kv_heads=hkv, head_dim=d, seq_len=t, seed=630 + t, dtype=dtype)
    pk, pv, table, _, _ = _paged_case(inp, bs, 631 + t)
    g = torch.Generator().manual_seed(632 + t)
    k_new = torch.randn(b, hkv, d, generator=g).to("cuda", dtype)
    v_new = torch.randn(b, hkv, d, generator=g).to("cuda", dtype)
    pk2, pv2 = pk.clone(), pv.clone()
    blk = table[:, (t - 1) // bs].long()
    pk2[blk, (t - 1) % bs] = k_new
    pv2[blk, (t - 1) % bs] = v_new
    want = mk.full_attention_decode(mk.FullAttentionInputs(inp.q, pk2, pv2, scale=inp.scale, block_table=table,
                                                           seq_len=t))
    got = mk.full_attention_decode(mk.FullAttentionInputs(inp.q, pk, pv, scale=inp.scale, block_table=table,
                                                          seq_len=t, k_new=k_new, v_new=v_new))
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(pk, pk2) and torch.equal(pv, pv2)


@pytest.mark.parametrize("b,hq,hkv,d,t,bs,rot,dtype", [
    (1, 24, 4, 256, 32768, 16, 64, torch.bfloat16),   # config 4 with RoPE, 16-token blocks
    (3, 8, 2, 128, 3001, 64, 32, torch.float16),
    (2, 8, 2, 128, 300, 32, 24, torch.bfloat16),      # rotary_dim the kernel cannot rotate: gathered first
])
def test_attention_paged_rope_equals_contiguous_rope(b, hq, hkv, d, t, bs, rot, dtype):
    """Paged KV with RoPE: bit-identical to the contiguous RoPE path on the
    same tokens (keys rotated in the kernel where it can, else gathered and
    rotated as the reference does)."""
    inp = make_attention(batch=b, q_heads=hq, kv_heads=hkv, head_dim=d, seq_len=t, seed=640 + t, dtype=dtype)
    pk, pv, table, _, _ = _paged_case(inp, bs, 641 + t)
    ang = torch.rand(rot, generator=torch.Generator().manual_seed(642)) * 6.0
    cos, sin = torch.cos(ang)[None], torch.sin(ang)[None]
    want = mk.full_attention_decode(mk.FullAttentionInputs(inp.q, inp.k_cache, inp.v_cache, cos=cos, sin=sin,
                                                           rotary_dim=rot, scale=inp.scale))
    got = mk.full_attention_decode(mk.FullAttentionInputs(inp.q, pk, pv, cos=cos, sin=sin, rotary_dim=rot,
                                                          scale=inp.scale, block_table=table, seq_len=t))
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("b,hq,hkv,d,t,bs,rot,dtype", [
    (1, 24, 4, 256, 32768, 16, 64, torch.bfloat16),   # config 4 with RoPE and the append, 16-token blocks
    (3, 8, 2, 128, 3001, 64, 32, torch.float16),      # ragged last block
    (2, 40, 2, 128, 1, 16, 128, torch.bfloat16),      # the first token of a fresh block; group 20; full rotation
])
def test_attention_paged_append_rope_equals_write_then_attend(b, hq, hkv, d, t, bs, rot, dtype):
    """Paged KV with both the append and RoPE in one launch: the output and
    both pools are bit-identical to writing the unrotated new row into its
    block with torch and then running the paged RoPE kernel; no other row
    changes."""
    inp = make_attention(batch=b, q_heads=hq, kv_heads=hkv, head_dim=d, seq_len=t, seed=650 + t, dtype=dtype)
    pk, pv, table, _, _ = _paged_case(inp, bs, 651 + t)
    g = torch.Generator().manual_seed(652 + t)
    k_new = torch.randn(b, hkv, d, generator=g).to("cuda", dtype)
    v_new = torch.randn(b, hkv, d, generator=g).to("cuda", dtype)
    ang = torch.rand(rot, generator=g) * 6.0
    cos, sin = torch.cos(ang)[None], torch.sin(ang)[None]
    pk2, pv2 = pk.clone(), pv.clone()
    blk = table[:, (t - 1) // bs].long()
    pk2[blk, (t - 1) % bs] = k_new
    pv2[blk, (t - 1) % bs] = v_new
    want = mk.full_attention_decode(mk.FullAttentionInputs(inp.q, pk2, pv2, cos=cos, sin=sin, rotary_dim=rot,
                                                           scale=inp.scale, block_table=table, seq_len=t))
    got = mk.full_attention_decode(mk.FullAttentionInputs(inp.q, pk, pv, cos=cos, sin=sin, rotary_dim=rot,
                                                          scale=inp.scale, block_table=table, seq_len=t,
                                                          k_new=k_new, v_new=v_new))
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(pk, pk2) and torch.equal(pv, pv2)


def test_attention_paged_append_rope_graph_replay():
    """Paged KV with the append and RoPE in one launch, captured in a HIP
    graph: every replay writes the same row and returns the eager output bit
    for bit, with an eager contiguous call sharing the workspace between
    replays."""
    t, bs, rot = 4096, 16, 64
    inp = make_attention(seq_len=t, seed=671)
    pk, pv, table, _, _ = _paged_case(inp, bs, 672)
    g = torch.Generator().manual_seed(673)
    k_new = torch.randn(1, 4, 256, generator=g).to("cuda", torch.bfloat16)
    v_new = torch.randn(1, 4, 256, generator=g).to("cuda", torch.bfloat16)
    ang = torch.rand(rot, generator=g) * 6.0
    cos, sin = torch.cos(ang)[None], torch.sin(ang)[None]
    args = mk.FullAttentionInputs(inp.q, pk, pv, cos=cos, sin=sin, rotary_dim=rot, scale=inp.scale,
                                  block_table=table, seq_len=t, k_new=k_new, v_new=v_new)
    eager = mk.full_attention_decode(args)
    pk_e, pv_e = pk.clone(), pv.clone()
    other = make_attention(batch=1, q_heads=8, kv_heads=2, head_dim=128, seq_len=3000, seed=674)
    other_ref = mk.full_attention_decode(other)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mk.full_attention_decode(args)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        res = mk.full_attention_decode(args)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(res, eager)
        assert torch.equal(pk, pk_e) and torch.equal(pv, pv_e)
        with torch.cuda.stream(s):
            mid = mk.full_attention_decode(other)
        torch.cuda.synchronize()
        assert torch.equal(mid, other_ref)
