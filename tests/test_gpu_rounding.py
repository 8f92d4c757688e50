"""bf16 rounding of FP32 results: round to nearest, ties to even.

Every kernel rounds its FP32 results to bf16 through one helper pair
(``f2bf_bits`` / ``f2bf2_bits`` in csrc/mkq_device.h, the compiler's float to
__bf16 conversion).  These cases reach it through the projection GEMV
(``mkq_gemv``): with one nonzero weight per output row, y[i] = bf16(x[i] * s[i]),
and the FP32 product of two bf16 factors is exact, so the output's only rounding
is the helper's.  The products are chosen to hit ties with an even and with an
odd last bit, values just above and below a tie, the tie at the largest finite
bf16 (which rounds to infinity), and FP32 denormals that need rounding.  The
expected bits come from the integer rule (u + 0x7fff + lsb) >> 16, which torch's
CPU conversion is checked against here as well.
"""

import numpy as np
import pytest
import torch

import mega_kernel_qwen36 as mk

pytestmark = pytest.mark.gpu


def _rne_bits(p32: np.ndarray) -> np.ndarray:
    u = p32.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _bf16(v: float) -> np.float32:
    """v as a bf16-representable float32 (v must be one)."""
    f = np.float32(v)
    assert (f.view(np.uint32) & 0xFFFF) == 0, v
    return f


def _cases():
    """(x, s) bf16 pairs whose exact FP32 product needs each kind of rounding."""
    rng = np.random.default_rng(7)
    want = {"tie_even": 4, "tie_odd": 4, "above_tie": 4, "below_tie": 4, "exact": 2}
    got = {k: [] for k in want}
    while any(len(got[k]) < n for k, n in want.items()):
        xb = rng.integers(0x3E00, 0x4200, dtype=np.uint32) | (rng.integers(0, 2, dtype=np.uint32) << 15)
        sb = rng.integers(0x3E00, 0x4200, dtype=np.uint32)
        x = np.uint32(xb << 16).view(np.float32)
        s = np.uint32(sb << 16).view(np.float32)
        p = np.float64(x) * np.float64(s)
        p32 = np.float32(p)
        assert np.float64(p32) == p  # two 8-bit significands: the product is exact
        lo = int(p32.view(np.uint32)) & 0xFFFF
        odd = (int(p32.view(np.uint32)) >> 16) & 1
        kind = ("exact" if lo == 0 else "tie_odd" if lo == 0x8000 and odd else "tie_even" if lo == 0x8000
                else "above_tie" if lo > 0x8000 else "below_tie")
        if len(got[kind]) < want[kind]:
            got[kind].append((x, s))
    pairs = [p for k in want for p in got[k]]
    # the tie at the largest finite bf16 (0x7f7f, odd): (511/256) * 2^127 rounds to +inf
    pairs.append((_bf16(1.75), _bf16(73 / 64 * 2.0 ** 127)))
    pairs.append((_bf16(-1.75), _bf16(73 / 64 * 2.0 ** 127)))
    # FP32 denormal products: 31 * 2^-134 is a tie between bf16 denormals 15 and 16 (units of 2^-133)
    pairs.append((_bf16(31 / 16 * 2.0 ** -100), _bf16(2.0 ** -30)))
    pairs.append((_bf16(-29 / 16 * 2.0 ** -100), _bf16(2.0 ** -30)))
    pairs.append((_bf16(1.5 * 2.0 ** -100), _bf16(1.25 * 2.0 ** -30)))
    return pairs


def test_gemv_output_rounding_matches_round_to_nearest_even():
    pairs = _cases()
    n = 64  # 16-byte rows of 8 chunks: the vector GEMV path
    assert len(pairs) <= n
    x = np.zeros(n, np.float32)
    s = np.zeros(n, np.float32)
    for i, (xi, si) in enumerate(pairs):
        x[i], s[i] = xi, si
    p32 = (x.astype(np.float64) * s.astype(np.float64)).astype(np.float32)
    want = _rne_bits(p32)
    # torch's CPU conversion agrees with the rule on every case
    torch_bits = torch.from_numpy(p32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(torch_bits, want)
    # the cases cover both tie directions, infinity and a denormal tie
    assert 0x7F80 in want and 0xFF80 in want and 0x0010 in want

    dev = torch.device("cuda")
    xt = torch.from_numpy(x).to(torch.bfloat16).reshape(1, n).to(dev)
    w = torch.diag(torch.from_numpy(s)).to(torch.bfloat16).to(dev).contiguous()
    assert torch.equal(xt.float().cpu().reshape(-1), torch.from_numpy(x))
    assert torch.equal(torch.diagonal(w.float().cpu()), torch.from_numpy(s))
    y = mk.ops._C.gemv(xt, w, None)
    torch.cuda.synchronize()
    got = y.reshape(-1).view(torch.int16).cpu().numpy().view(np.uint16)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(int(i), hex(int(p32[i].view(np.uint32))), hex(int(got[i])), hex(int(want[i]))) for i in bad]
