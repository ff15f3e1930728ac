"""Seeded random decode shapes (1 - 64 rows; and 1 - 6 rows on deep rows of
wide outputs) through the launchers that use
the weight-streaming kernel of csrc/w8a16_stream.h: the W8A16 linear and its
int8 gate/up + SiLU-and-mul, the 16-bit linear and the 16-bit gate/up +
SiLU-and-mul.  Their launch plans (rows per workgroup, 4-row weight and x
sets, waves, chunks in flight) are picked per call from the row count, k,
the output width and the CU count, and rows, k and n are drawn so that the
picks vary: ragged last workgroups, partial last chunks of K, x tiles
padded past the last row, and some x passed as a row-strided view.

Each shape is checked against fp64 GEMMs on the GPU: the fp32 output within
the worst-case fp32 summation error (gamma_k * sum |x w|, carried through
SiLU-and-mul where it applies), the 16-bit output within one output ulp
more, and the 16-bit output equal to the fp32 output rounded once.
"""
import numpy as np
import pytest
import torch

from parity_utils import act_error_bound, gen, ulp16

pytestmark = pytest.mark.gpu

F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32


def _shapes(seed, count, rows, k_step, k_max, n_max):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        out.append((int(rng.integers(rows[0], rows[1] + 1)), int(rng.integers(1, k_max // k_step + 1)) * k_step,
                    int(rng.integers(1, n_max + 1)), F16 if i % 2 == 0 else BF16, bool(rng.integers(0, 2))))
    return out


def _deep_shapes(seed, count, rows, k_step):
    """A few rows on deep rows of wide outputs (k 3072 - 12000, n 4100 -
    12000, n k <= 6e7): the 16-row workgroups of one x set and the dual
    kernel's 8-row workgroups of 8 waves."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        r, k, n = int(rng.integers(rows[0], rows[1] + 1)), int(rng.integers(3072 // k_step, 12000 // k_step + 1)) * k_step, \
            int(rng.integers(4100, 12001))
        if n * k <= 6e7:
            out.append((r, k, n, F16 if len(out) % 2 == 0 else BF16, bool(rng.integers(0, 2))))
    return out


# (rows, k, n, dtype, x as a row-strided view); n below 8192 keeps the small
# tiled shapes of 17 - 64 rows out, so every case takes the stream kernel
W8A16 = _shapes(3031, 12, (1, 48), 16, 4096, 4000) + _deep_shapes(3035, 6, (1, 4), 16)
W8A16_DUAL = _shapes(3032, 10, (1, 32), 16, 4096, 4000) + _deep_shapes(3036, 4, (2, 4), 16)
LINEAR16 = _shapes(3033, 12, (1, 64), 8, 4096, 4000) + _deep_shapes(3037, 4, (3, 6), 8)
GATE_UP16 = _shapes(3034, 10, (1, 32), 8, 4096, 4000)


def _x(rows, k, dt, seed, cuda, strided):
    x = torch.randn(rows, k, generator=gen(seed)).to(dt)
    if not strided:
        return x.to(cuda)
    big = torch.zeros(rows, k + 24, dtype=dt)
    big[:, 8:8 + k] = x
    return big.to(cuda)[:, 8:8 + k]   # row stride k + 24, 16-byte aligned rows


def _w(n, k, dt, seed, std, cuda):
    return (torch.randn(n, k, generator=gen(seed)) * std).to(dt).to(cuda)


def _gamma(k):
    return k * 2.0 ** -24 / (1 - k * 2.0 ** -24)


def _check_linear(got16, got32, exact, bound, dt):
    ulp = torch.from_numpy(ulp16(exact.cpu().numpy(), dt)).to(exact.device)
    got32 = got32.double()
    assert float(((got32 - exact).abs() - (bound + 2.0 ** -23 * exact.abs() + 1e-30)).max()) <= 0
    assert float(((got16.double() - exact).abs() - (ulp + bound + 2.0 ** -22 * exact.abs())).max()) <= 0
    assert torch.equal(got16, got32.to(got16.dtype)), "the 16-bit output must be the fp32 output rounded once"


def _check_act(got16, got32, g, u, gabs, uabs, k, dt):
    exact = torch.nn.functional.silu(g) * u
    bound = torch.from_numpy(act_error_bound(g.cpu().numpy(), u.cpu().numpy(), gabs.cpu().numpy(),
                                             uabs.cpu().numpy(), k)).to(g.device)
    ulp = torch.from_numpy(ulp16(exact.cpu().numpy(), dt)).to(g.device)
    got16, got32 = got16.double(), got32.double()
    assert float(((got32 - exact).abs() - (2.0 ** -22 * exact.abs() + bound)).max()) <= 1e-30
    assert float(((got16 - exact).abs() - (ulp + bound + 2.0 ** -22 * exact.abs())).max()) <= 0
    assert torch.equal(got16.to(dt), got32.to(dt)), "the 16-bit output must be the fp32 output rounded once"


@pytest.mark.parametrize("rows,k,n,dt,strided", W8A16)
def test_w8a16_random_decode_shapes(pkg, cuda, rows, k, n, dt, strided):
    x = _x(rows, k, dt, rows + k, cuda, strided)
    q, sc = pkg.quantize_int8_weight(_w(n, k, dt, n, k ** -0.5, cuda))
    got16 = pkg.w8a16_linear(x, q, sc)
    got32 = pkg.w8a16_linear(x, q, sc, out_dtype=F32)
    x64, q64, s64 = x.double(), q.double(), sc.double()
    _check_linear(got16, got32, (x64 @ q64.T) * s64, _gamma(k) * (x64.abs() @ q64.abs().T) * s64.abs(), dt)


@pytest.mark.parametrize("rows,k,n,dt,strided", W8A16_DUAL)
def test_gate_up_silu_w8a16_random_decode_shapes(pkg, cuda, rows, k, n, dt, strided):
    x = _x(rows, k, dt, rows + k, cuda, strided)
    qg, sg = pkg.quantize_int8_weight(_w(n, k, dt, n, 2.0 * k ** -0.5, cuda))
    qu, su = pkg.quantize_int8_weight(_w(n, k, dt, n + 1, k ** -0.5, cuda))
    got16 = pkg.fused_gate_up_silu_w8a16(x, qg, sg, qu, su)
    got32 = pkg.fused_gate_up_silu_w8a16(x, qg, sg, qu, su, out_dtype=F32)
    x64 = x.double()
    g64, u64 = qg.double(), qu.double()
    sg64, su64 = sg.double(), su.double()
    _check_act(got16, got32, (x64 @ g64.T) * sg64, (x64 @ u64.T) * su64, (x64.abs() @ g64.abs().T) * sg64.abs(),
               (x64.abs() @ u64.abs().T) * su64.abs(), k, dt)


@pytest.mark.parametrize("rows,k,n,dt,strided", LINEAR16)
def test_linear16_random_decode_shapes(pkg, cuda, rows, k, n, dt, strided):
    x = _x(rows, k, dt, rows + k, cuda, strided)
    w = _w(n, k, dt, n, k ** -0.5, cuda)
    b = (torch.randn(n, generator=gen(n + 7)) * 0.1).to(dt).to(cuda) if rows % 2 else None
    got16 = pkg.linear16(x, w, b)
    got32 = pkg.linear16(x, w, b, out_dtype=F32)
    x64, w64 = x.double(), w.double()
    exact = x64 @ w64.T + (b.double() if b is not None else 0.0)
    _check_linear(got16, got32, exact, _gamma(k) * (x64.abs() @ w64.abs().T), dt)


@pytest.mark.parametrize("rows,k,n,dt,strided", GATE_UP16)
def test_gate_up_silu_random_decode_shapes(pkg, cuda, rows, k, n, dt, strided):
    x = _x(rows, k, dt, rows + k, cuda, strided)
    wg, wu = _w(n, k, dt, n, 2.0 * k ** -0.5, cuda), _w(n, k, dt, n + 1, k ** -0.5, cuda)
    got16 = pkg.fused_gate_up_silu(x, wg, wu)
    got32 = pkg.fused_gate_up_silu(x, wg, wu, out_dtype=F32)
    x64, g64, u64 = x.double(), wg.double(), wu.double()
    _check_act(got16, got32, x64 @ g64.T, x64 @ u64.T, x64.abs() @ g64.abs().T, x64.abs() @ u64.abs().T, k, dt)
