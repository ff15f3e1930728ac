"""Broadcast and overlapping inputs to the projection launchers.

The reference's W8A16 launcher flattens its input with
``x.reshape(-1, K).contiguous()`` (src/kernels/w8a16_matmul_triton.py:
117-118), so a broadcast activation (``expand()``: row stride 0) works.  The
kernels here stream rows through row strides, which must be at least K; the
launchers therefore copy such views (and weights with overlapping rows)
before the call.  Each launcher's result on the broadcast view must equal its
result on the same values laid out contiguously, bit for bit.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

F16 = torch.float16


def _gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _x_broadcast(rows, k, cuda):
    row = torch.randn(1, k, generator=_gen(1)).to(F16).to(cuda)
    x = row.expand(rows, k)
    assert x.stride(0) == 0
    return x


@pytest.mark.parametrize("rows", [4, 300])  # skinny and tiled kernels
def test_w8a16_and_linear16_broadcast_x(pkg, cuda, rows):
    k, n = 1536, 2048
    x = _x_broadcast(rows, k, cuda)
    w = (0.02 * torch.randn(n, k, generator=_gen(2))).to(F16).to(cuda)
    bias = torch.randn(n, generator=_gen(3)).to(F16).to(cuda)
    q, scale = pkg.quantize_int8_weight(w)
    assert torch.equal(pkg.w8a16_linear(x, q, scale, bias), pkg.w8a16_linear(x.contiguous(), q, scale, bias))
    assert torch.equal(pkg.linear16(x, w, bias), pkg.linear16(x.contiguous(), w, bias))


@pytest.mark.parametrize("rows", [4, 300])
def test_gate_up_launchers_broadcast_x(pkg, cuda, rows):
    k, n = 1536, 2048
    x = _x_broadcast(rows, k, cuda)
    wg = (0.02 * torch.randn(n, k, generator=_gen(4))).to(F16).to(cuda)
    wu = (0.02 * torch.randn(n, k, generator=_gen(5))).to(F16).to(cuda)
    assert torch.equal(pkg.fused_gate_up_silu(x, wg, wu), pkg.fused_gate_up_silu(x.contiguous(), wg, wu))
    qg, sg = pkg.quantize_int8_weight(wg)
    qu, su = pkg.quantize_int8_weight(wu)
    assert torch.equal(pkg.fused_gate_up_silu_w8a16(x, qg, sg, qu, su),
                       pkg.fused_gate_up_silu_w8a16(x.contiguous(), qg, sg, qu, su))


def test_weights_with_overlapping_rows(pkg, cuda):
    """A weight whose rows overlap (row stride below K) is copied by the
    launcher, not handed to the kernel as is."""
    k, n = 1536, 256
    x = torch.randn(8, k, generator=_gen(6)).to(F16).to(cuda)
    w_row = (0.02 * torch.randn(1, k, generator=_gen(7))).to(F16).to(cuda)
    w = w_row.expand(n, k)
    assert torch.equal(pkg.linear16(x, w), pkg.linear16(x, w.contiguous()))
    q_row, s_row = pkg.quantize_int8_weight(w_row)
    q, s = q_row.expand(n, k), s_row.expand(n)
    assert torch.equal(pkg.w8a16_linear(x, q, s), pkg.w8a16_linear(x, q.contiguous(), s.contiguous()))
    assert torch.equal(pkg.fused_gate_up_silu(x, w, w), pkg.fused_gate_up_silu(x, w.contiguous(), w.contiguous()))
