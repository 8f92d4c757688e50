"""mkq_moe_decode_noalloc through the C ABI: the MoE decode with its workspace
in a static device array instead of a caller workspace.  Each call must give
the same indices, weights and output, bit for bit, as mkq_moe_decode on the
same inputs with a workspace of its own; two calls in a row, the second with
a smaller batch (a different kernel instance over the same array), and a
third repeating the first shape after it."""

import pytest
import torch

from mega_kernel_qwen36 import _lib
from tests.inputs import make_moe

FIELDS = ("norm_weight", "router_weight", "expert_gate", "expert_up", "expert_down", "shared_gate", "shared_up",
          "shared_down", "shared_expert_gate")


def _outputs(batch, hidden, top_k, dtype):
    return (torch.empty(batch, hidden, dtype=dtype, device="cuda"),
            torch.empty(batch, top_k, dtype=torch.int64, device="cuda"),
            torch.empty(batch, top_k, dtype=torch.float32, device="cuda"))


def _call(lib, x, w, top_k, noalloc):
    batch, hidden = x.shape
    experts, inter = w.expert_gate.shape[0], w.expert_gate.shape[1]
    shared = w.shared_gate.shape[0]
    out, idx, wts = _outputs(batch, hidden, top_k, x.dtype)
    ptrs = [getattr(w, n).data_ptr() for n in FIELDS]
    stream = torch.cuda.current_stream().cuda_stream
    head = (_lib.MKQ_DTYPE_BF16, x.data_ptr(), *ptrs, out.data_ptr(), idx.data_ptr(), wts.data_ptr(),
            batch, hidden, experts, inter, shared, top_k, 1e-6, 1)
    if noalloc:
        rc = lib.mkq_moe_decode_noalloc(*head, stream)
        ws = None
    else:
        nbytes = lib.mkq_moe_decode_workspace_bytes(batch, hidden, experts, inter, shared, top_k)
        ws = torch.zeros(nbytes + 256, dtype=torch.uint8, device="cuda")
        base = (ws.data_ptr() + 255) // 256 * 256
        rc = lib.mkq_moe_decode(*head, base, nbytes, stream)
    assert rc == _lib.MKQ_OK, lib.mkq_last_error()
    torch.cuda.synchronize()
    del ws
    return out, idx, wts


@pytest.mark.gpu
def test_noalloc_moe_matches_workspace_entry_point():
    lib = _lib.load_library()
    _, w, k = make_moe(batch=1, seed=401)
    for batch, seed in ((4, 402), (1, 403), (4, 404)):
        print(f"noalloc MoE: config 2, batch {batch}, seed {seed}", flush=True)
        x = torch.randn(batch, 2048, generator=torch.Generator().manual_seed(seed)).to("cuda", torch.bfloat16)
        got = _call(lib, x, w, k, noalloc=True)
        want = _call(lib, x, w, k, noalloc=False)
        assert torch.equal(got[1], want[1]), "top-k indices differ"
        assert torch.equal(got[2], want[2]), "route weights differ"
        assert torch.equal(got[0], want[0]), "outputs differ"
        assert torch.isfinite(got[0].float()).all()
