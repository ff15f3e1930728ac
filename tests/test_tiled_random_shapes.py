"""Seeded random prefill shapes through the tiled MFMA GEMM launchers, whose
launch plans (tile shape, step pipeline or sub-step ring, column split) are
picked per call from the row count, the output width and the CU count.

Each shape is checked against fp64 GEMMs on the GPU: the 16-bit output
within one output ulp plus the worst-case fp32 summation error (gamma_k *
sum |x w|, carried through SiLU-and-mul where it applies), the fp32 output
within that bound, and the 16-bit output equal to the fp32 output rounded
once.  Rows, k (a multiple of the path's alignment) and n are drawn
uniformly, so ragged row blocks, k tails and ragged column blocks meet every
plan the launchers can choose at these sizes.
"""
import numpy as np
import pytest
import torch

from parity_utils import act_error_bound, gen, ulp16

pytestmark = pytest.mark.gpu

F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32


def _shapes(seed, count, rows, k_step, k_max, n):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        out.append((int(rng.integers(rows[0], rows[1] + 1)), int(rng.integers(1, k_max // k_step + 1)) * k_step,
                    int(rng.integers(n[0], n[1] + 1)), F16 if i % 2 == 0 else BF16))
    return out


GATE_UP = _shapes(2024, 8, (129, 2200), 8, 600, (1, 9500))
W8A16 = _shapes(2025, 8, (129, 4200), 16, 600, (2049, 9000))
W8A16_DUAL = _shapes(2026, 6, (257, 2200), 16, 600, (64, 19000))


def _x(rows, k, dt, seed, cuda):
    return torch.randn(rows, k, generator=gen(seed)).to(dt).to(cuda)


def _w(n, k, dt, seed, std, cuda):
    return (torch.randn(n, k, generator=gen(seed)) * std).to(dt).to(cuda)


def _check_act(got16, got32, g, u, gabs, uabs, k, dt):
    exact = torch.nn.functional.silu(g) * u
    bound = torch.from_numpy(act_error_bound(g.cpu().numpy(), u.cpu().numpy(), gabs.cpu().numpy(),
                                             uabs.cpu().numpy(), k)).to(g.device)
    ulp = torch.from_numpy(ulp16(exact.cpu().numpy(), dt)).to(g.device)
    got16, got32 = got16.double(), got32.double()
    assert float(((got32 - exact).abs() - (2.0 ** -22 * exact.abs() + bound)).max()) <= 1e-30
    assert float(((got16 - exact).abs() - (ulp + bound + 2.0 ** -22 * exact.abs())).max()) <= 0
    assert torch.equal(got16.to(dt), got32.to(dt)), "the 16-bit output must be the fp32 output rounded once"


@pytest.mark.parametrize("rows,k,n,dt", GATE_UP)
def test_gate_up_silu_random_prefill_shapes(pkg, cuda, rows, k, n, dt):
    x = _x(rows, k, dt, rows + k, cuda)
    wg, wu = _w(n, k, dt, n, 2.0 * k ** -0.5, cuda), _w(n, k, dt, n + 1, k ** -0.5, cuda)
    got16 = pkg.fused_gate_up_silu(x, wg, wu)
    got32 = pkg.fused_gate_up_silu(x, wg, wu, out_dtype=F32)
    x64, g64, u64 = x.double(), wg.double(), wu.double()
    _check_act(got16, got32, x64 @ g64.T, x64 @ u64.T, x64.abs() @ g64.abs().T, x64.abs() @ u64.abs().T, k, dt)


@pytest.mark.parametrize("rows,k,n,dt", W8A16)
def test_w8a16_random_prefill_shapes(pkg, cuda, rows, k, n, dt):
    x = _x(rows, k, dt, rows + k, cuda)
    q, sc = pkg.quantize_int8_weight(_w(n, k, dt, n, k ** -0.5, cuda))
    got16 = pkg.w8a16_linear(x, q, sc)
    got32 = pkg.w8a16_linear(x, q, sc, out_dtype=F32).double()
    x64, q64, s64 = x.double(), q.double(), sc.double()
    exact = (x64 @ q64.T) * s64
    gam = k * 2.0 ** -24 / (1 - k * 2.0 ** -24)
    bound = gam * (x64.abs() @ q64.abs().T) * s64.abs()
    ulp = torch.from_numpy(ulp16(exact.cpu().numpy(), dt)).to(cuda)
    assert float(((got32 - exact).abs() - (bound + 2.0 ** -23 * exact.abs() + 1e-30)).max()) <= 0
    assert float(((got16.double() - exact).abs() - (ulp + bound + 2.0 ** -22 * exact.abs())).max()) <= 0
    assert torch.equal(got16, got32.to(dt)), "the 16-bit output must be the fp32 output rounded once"


@pytest.mark.parametrize("rows,k,n,dt", W8A16_DUAL)
def test_gate_up_silu_w8a16_random_prefill_shapes(pkg, cuda, rows, k, n, dt):
    x = _x(rows, k, dt, rows + k, cuda)
    qg, sg = pkg.quantize_int8_weight(_w(n, k, dt, n, 2.0 * k ** -0.5, cuda))
    qu, su = pkg.quantize_int8_weight(_w(n, k, dt, n + 1, k ** -0.5, cuda))
    got16 = pkg.fused_gate_up_silu_w8a16(x, qg, sg, qu, su)
    got32 = pkg.fused_gate_up_silu_w8a16(x, qg, sg, qu, su, out_dtype=F32)
    x64 = x.double()
    qg64, qu64, sg64, su64 = qg.double(), qu.double(), sg.double(), su.double()
    _check_act(got16, got32, (x64 @ qg64.T) * sg64, (x64 @ qu64.T) * su64,
               (x64.abs() @ qg64.abs().T) * sg64.abs(), (x64.abs() @ qu64.abs().T) * su64.abs(), k, dt)
