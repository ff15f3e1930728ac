"""GPU checks of the weight-only int8 linear (``mi355_w8a16_linear_fwd``) and
its quantiser (``mi355_quantize_int8_fwd``), after the reference's
tests/test_w8a16_kernel.py (same layer shapes, M values, bias cases,
tolerances and quantisation-error bounds), with the CPU oracle as the checker:

* the HIP quantiser equals the oracle's restatement of
  QuantizedLinearInt8.from_linear bit for bit (int8 codes and fp32 scales),
  at every shape used here;
* the kernel's output is the exact value (fp64) within one output ulp plus
  the worst-case fp32 summation error gamma_k * scale * sum|x * q|, for every
  output (against an fp64 GEMM of the same int8 weights on the GPU); >= 99%
  of the outputs equal the oracle's single-rounding result bit for bit (on
  a column sample for the large shapes, whole outputs otherwise); the fp32
  output sits within the same bound; and the reference's own check against
  its dequantise-first reference (atol = rtol = 2e-2) holds;
* decode (<= 32 rows), prefill (tiled) and generic (odd k / misaligned)
  kernels, fp16 and bf16, fp32 / fp16 / bf16 scales and biases, strided and
  3-D inputs, row-strided outputs, graph replay, determinism, Qwen2.5-7B
  shapes.
"""
import importlib

import numpy as np
import pytest
import torch

from parity_utils import DT_NAME, gen, storage

pytestmark = pytest.mark.gpu

F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32

# (K = in_features, N = out_features), as in the reference's test
LAYER_SHAPES = [
    (1536, 1536),   # q_proj / o_proj
    (1536, 256),    # k_proj / v_proj (2 KV heads x 128)
    (1536, 8960),   # gate_proj / up_proj
    (8960, 1536),   # down_proj
    (100, 37),      # awkward: not a multiple of any block size
]
M_VALUES = [1, 7, 16, 100, 300]


def _linear(K, N, bias, cuda, dtype=F16, seed=0):
    g = gen(seed)
    lin = torch.nn.Linear(K, N, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g) * 0.05)
        if bias:
            lin.bias.copy_(torch.randn(N, generator=g) * 0.1)
    return lin.to(device=cuda, dtype=dtype)


def _x(M, K, dtype, cuda, seed=1):
    return torch.randn(M, K, generator=gen(seed)).to(dtype).to(cuda)


def _ulp(v: np.ndarray, dt) -> np.ndarray:
    mant, emin = (10, -14) if dt == F16 else (7, -126)
    e = np.maximum(np.floor(np.log2(np.maximum(np.abs(v), 1e-300))), emin)
    return 2.0 ** (e - mant)


def _check_quantizer(orc, lin, q):
    wdt = DT_NAME[lin.weight.dtype]
    oq, osc = orc.quantize_int8(storage(lin.weight.detach()), wdt=wdt)
    assert np.array_equal(q.weight_q.cpu().numpy(), oq), "int8 codes differ from the oracle"
    assert np.array_equal(q.scale.cpu().numpy().view(np.uint32), osc.view(np.uint32)), "scales differ"


def _check_kernel(orc, x, q, got16, got32, max_oracle_macs=2e7):
    """got16 / got32: the kernel's outputs (x dtype / fp32), [M, N] on the GPU."""
    M, K = x.shape
    N = q.weight_q.shape[0]
    k_gamma = K * 2.0 ** -24 / (1 - K * 2.0 ** -24)
    x64, q64 = x.double(), q.weight_q.double()
    sc = q.scale.double()
    exact = (x64 @ q64.T) * sc
    if q.bias is not None:
        exact = exact + q.bias.double()
    bound = k_gamma * (x64.abs() @ q64.abs().T) * sc.abs()
    ex = exact.cpu().numpy()
    bd = bound.cpu().numpy()
    g16 = got16.double().cpu().numpy()
    tol16 = _ulp(ex, x.dtype) + bd + 2.0 ** -22 * np.abs(ex)
    assert np.all(np.abs(g16 - ex) <= tol16), f"max excess {np.max(np.abs(g16 - ex) - tol16):.3e}"
    g32 = got32.double().cpu().numpy()
    assert np.all(np.abs(g32 - ex) <= bd + 2.0 ** -23 * np.abs(ex) + 1e-30), "fp32 output outside the bound"

    # bit-equality with the oracle's single-rounding result, on a column sample for large shapes
    ncols = int(max(8, min(N, max_oracle_macs // max(1, M * K))))
    cols = np.unique(np.linspace(0, N - 1, ncols).round().astype(np.int64))
    name = DT_NAME[x.dtype]
    bias = None if q.bias is None else storage(q.bias[cols].cpu())
    r = orc.w8a16_linear(storage(x.cpu()), q.weight_q[cols].cpu().numpy(), q.scale[cols].cpu().numpy(), bias,
                         xdt=name, bdt=None if q.bias is None else DT_NAME[q.bias.dtype])
    assert np.allclose(r["out64"], ex[:, cols], rtol=1e-12, atol=1e-12)
    same = float(np.mean(storage(got16.cpu())[:, cols] == r["out"]))
    assert same >= 0.99, f"only {same:.4f} of outputs equal the oracle's single rounding"
    return same


@pytest.mark.parametrize("K,N", LAYER_SHAPES)
@pytest.mark.parametrize("M", M_VALUES)
@pytest.mark.parametrize("bias", [False, True])
def test_kernel_matches_dequantized_reference(pkg, orc, cuda, K, N, M, bias):
    lin = _linear(K, N, bias, cuda)
    q = pkg.QuantizedLinearInt8.from_linear(lin)
    _check_quantizer(orc, lin, q)
    x = _x(M, K, F16, cuda)

    kernel_out = pkg.w8a16_linear(x, q.weight_q, q.scale, q.bias)
    ref_out = pkg.w8a16_reference(x, q.weight_q, q.scale, q.bias)
    torch.testing.assert_close(kernel_out, ref_out, atol=2e-2, rtol=2e-2)   # the reference's bar
    got32 = pkg.w8a16_linear(x, q.weight_q, q.scale, q.bias, out_dtype=F32)
    assert kernel_out.dtype == F16 and kernel_out.shape == (M, N)
    _check_kernel(orc, x, q, kernel_out, got32)


@pytest.mark.parametrize("M,K,N,bias", [(1, 1536, 8960, False), (8, 3584, 512, True), (24, 896, 4864, True),
                                        (32, 1536, 256, False), (64, 1536, 1536, True), (300, 640, 200, False),
                                        (5, 100, 37, True), (1, 4864, 896, True)])
def test_bf16_matches_oracle(pkg, orc, cuda, M, K, N, bias):
    lin = _linear(K, N, bias, cuda, dtype=BF16, seed=M)
    q = pkg.QuantizedLinearInt8.from_linear(lin)
    _check_quantizer(orc, lin, q)
    x = _x(M, K, BF16, cuda, seed=M + 1)
    got16 = pkg.w8a16_linear(x, q.weight_q, q.scale, q.bias)
    got32 = pkg.w8a16_linear(x, q.weight_q, q.scale, q.bias, out_dtype=F32)
    same = _check_kernel(orc, x, q, got16, got32)
    print(f"bf16 W8A16 [{M}x{K}] x [{N}x{K}]: {same:.5f} equal to the oracle")


# Decode rows (<= 8: the lane-coalesced weight-streaming kernel) at every row
# count of an 8-row tile, over narrow outputs (fewer 8-row workgroups than CUs:
# 4-7 weight rows per workgroup), wide ones, a partial last 256-column chunk
# and a ragged last workgroup.
STREAM_CASES = [(m, K, N, F16 if (m + K) % 2 else BF16, m % 3 == 0)
                for m in range(1, 9)
                for K, N in ((8960, 1536), (1536, 8960), (272, 1000), (4864, 896), (1552, 37))]
# 9 - 16 rows: three or four 4-row x sets, and the wide, deep outputs the
# launcher keeps on the skinny kernel at 13 - 16 rows (n > 10000, k > 2048)
# and gives 16-row workgroups at 9 - 12 (k >= 3072), as it does k >= 3072
# with n > 2048 (here a partial last chunk and a ragged last workgroup)
STREAM_CASES += [(m, K, N, F16 if (m + K) % 2 else BF16, m % 2 == 0)
                 for m in (9, 12, 13, 16)
                 for K, N in ((8960, 1536), (1536, 8960), (272, 1000), (1552, 37), (3584, 10008))]
STREAM_CASES += [(m, 3104, 2900, F16 if m % 2 else BF16, m % 2 == 1) for m in (9, 10, 11, 12)]
# 1 - 4 rows on deep rows (k >= 3072) of outputs with at least a CU's worth
# of 16-row workgroups: 16-row workgroups (a partial last chunk and a ragged
# last workgroup at 3104 x 4204); below that (3104 x 2900) 8-row workgroups
STREAM_CASES += [(m, K, N, F16 if (m + K) % 2 else BF16, m % 2 == 1)
                 for m in (1, 2, 3, 4)
                 for K, N in ((3104, 4204), (3584, 10008), (3104, 2900))]
STREAM_CASES += [(3, 18944, 3584, BF16, False)]
# 49 - 64 rows of one matrix of at most 8 MB: 16 x sets, one 4-row weight set
# per workgroup (narrow outputs, a ragged last workgroup, a partial last chunk)
STREAM_CASES += [(56, 4864, 896, F16, True), (64, 1536, 1536, BF16, False), (60, 1552, 1002, F16, False)]
# beyond 16 rows from k = 2048: the 16-row class (balanced over the CUs; a
# ragged last workgroup and a partial last chunk at 2064 x 4204)
STREAM_CASES += [(20, 2048, 11008, F16, True), (28, 2064, 4204, BF16, False), (32, 2048, 6000, F16, False)]
# 17 - 32 rows where the small tiled shapes do not pay: 6 and 8 x sets
STREAM_CASES += [(m, K, N, F16 if (m + K) % 2 else BF16, m % 2 == 0)
                 for m in (17, 24, 25, 32)
                 for K, N in ((8960, 1536), (4864, 896), (3104, 2900), (1552, 37))]
# 33 - 48 rows (12 x sets, one matrix) where the small tiled shapes do not pay
STREAM_CASES += [(m, K, N, F16 if (m + K) % 2 else BF16, m % 2 == 1)
                 for m in (33, 48)
                 for K, N in ((8960, 1536), (3104, 2900), (1552, 37))]


@pytest.mark.parametrize("M,K,N,dt,bias", STREAM_CASES)
def test_decode_stream_kernel_matches_oracle(pkg, orc, cuda, M, K, N, dt, bias):
    lin = _linear(K, N, bias, cuda, dtype=dt, seed=M + K)
    q = pkg.QuantizedLinearInt8.from_linear(lin)
    x = _x(M, K, dt, cuda, seed=M + 5)
    got16 = pkg.w8a16_linear(x, q.weight_q, q.scale, q.bias)
    got32 = pkg.w8a16_linear(x, q.weight_q, q.scale, q.bias, out_dtype=F32)
    _check_kernel(orc, x, q, got16, got32)
    assert torch.equal(got16, got32.to(dt)), "the 16-bit output must be the fp32 output rounded once"


# Prefill shapes that land on each of the tiled GEMM's launch shapes (by the
# number of 128 x 128 output tiles), with k tails and ragged edges.
TILED_CASES = [
    (300, 1552, 1000, F16, True),     # < 128 tiles: 64 x 64
    (320, 512, 8960, F16, False),     # < 320: 128 x 128, 8 waves, step pipeline
    (200, 2048, 8960, BF16, True),    # <= 256 rows but a large grid: tiled, 128 x 128
    (4096, 256, 1536, F16, True),     # n <= 2048: 128 x 256
    (4096, 256, 1536, BF16, False),   # (bf16: 128 x 128)
    # n <= 2048 with between cus / 2 and cus tiles of 64 x 128: 8 waves, ring
    (1024, 1536, 1536, F16, True),    # 192 tiles
    (1000, 272, 2000, BF16, False),   # 256 tiles, ragged rows and n, k tail
    # n > 2048 below 1024 rows with >= 2 tiles of 128 x 64 per CU: the sub-step ring
    (512, 512, 8960, F16, False),     # 128 x 64, 4 waves (main loop and k tail)
    # n > 2048 from 1024 rows, k <= 4096: 128 x 128 tiles of 8 waves, 3-stage ring
    (2048, 128, 8952, F16, False),    # ragged n
    (4096, 64, 8960, F16, True),
    (4096, 80, 9000, BF16, True),     # ragged n, k tail only
    (4096, 32, 3584, BF16, True),
    # ... except where 192 x 128 tiles fit in one round of two workgroups per
    # CU and 128 x 128 tiles do not: 192 x 128, registers capped at 128
    (1024, 272, 8960, BF16, False),   # 420 tiles
    (1200, 400, 8000, F16, True),     # 441 tiles: ragged rows and n, k tail
    # n > 2048 with k > 4096 and many 128 x 64 tiles: the launch plan weighs
    # rounds of 128 x 64, 256 x 128 and 256 x 256 tiles (sub-step ring)
    (512, 4608, 14336, F16, True),    # 256 x 128, 8 waves of 128 x 32
    (1024, 4608, 14336, BF16, False), # 256 x 256, 8 waves of 64 x 128
    # 17 - 64 rows with >= 128 tile columns: the small tiled shapes
    (24, 1536, 8960, F16, True),      # 32 x 64
    (20, 256, 16400, BF16, False),    # n > 10000: 32 x 128
    (48, 272, 8200, F16, True),       # 33 - 64 rows: 64 x 64
]


@pytest.mark.parametrize("M,K,N,dt,bias", TILED_CASES)
def test_tiled_launch_shapes_match_oracle(pkg, orc, cuda, M, K, N, dt, bias):
    lin = _linear(K, N, bias, cuda, dtype=dt, seed=M + N)
    q = pkg.QuantizedLinearInt8.from_linear(lin)
    x = _x(M, K, dt, cuda, seed=M + 3)
    got16 = pkg.w8a16_linear(x, q.weight_q, q.scale, q.bias)
    got32 = pkg.w8a16_linear(x, q.weight_q, q.scale, q.bias, out_dtype=F32)
    same = _check_kernel(orc, x, q, got16, got32)
    assert torch.equal(got16, got32.to(dt)), "the 16-bit output must be the fp32 output rounded once"
    print(f"tiled W8A16 [{M}x{K}] x [{N}x{K}] {dt}: {same:.5f} equal to the oracle")


@pytest.mark.parametrize("M", [6, 14])
@pytest.mark.parametrize("sdt,bdt", [(F16, F16), (BF16, F32), (F32, BF16)])
def test_scale_and_bias_dtypes(pkg, orc, cuda, sdt, bdt, M):
    K, N = 512, 72
    lin = _linear(K, N, True, cuda, seed=4)
    q = pkg.QuantizedLinearInt8.from_linear(lin)
    x = _x(M, K, F16, cuda, seed=5)
    scale, bias = q.scale.to(sdt), q.bias.to(bdt)
    got = pkg.w8a16_linear(x, q.weight_q, scale, bias)
    r = orc.w8a16_linear(storage(x.cpu()), q.weight_q.cpu().numpy(), storage(scale.cpu()), storage(bias.cpu()),
                         xdt="f16", sdt=DT_NAME[sdt], bdt=DT_NAME[bdt])
    # every output within one ulp of the exact value plus the worst-case fp32
    # summation error of its k products (the kernel's summation order is its
    # own), and >= 99% equal to the oracle's single rounding
    ex = r["out64"]
    k_gamma = K * 2.0 ** -24 / (1 - K * 2.0 ** -24)
    sc = scale.double().cpu().numpy()
    tol = _ulp(ex, F16) + k_gamma * r["absacc"] * np.abs(sc) + 2.0 ** -22 * np.abs(ex)
    assert np.all(np.abs(got.double().cpu().numpy() - ex) <= tol)
    d = orc.ulp_diff16(storage(got.cpu()), r["out"])
    assert (d > 0).mean() < 0.01


def test_kernel_handles_3d_input(pkg, cuda):
    """Real model activations are (batch, seq, hidden), not 2D."""
    lin = _linear(1536, 256, True, cuda)
    q = pkg.QuantizedLinearInt8.from_linear(lin)
    x = torch.randn(2, 5, 1536, generator=gen(7)).to(F16).to(cuda)
    out = q(x)
    assert out.shape == (2, 5, 256)
    ref = pkg.w8a16_reference(x, q.weight_q, q.scale, q.bias)
    torch.testing.assert_close(out, ref, atol=2e-2, rtol=2e-2)
    assert torch.equal(out.view(10, 256), pkg.w8a16_linear(x.view(10, 1536), q.weight_q, q.scale, q.bias))


@pytest.mark.parametrize("K,N", [(1536, 1536), (1536, 8960)])
def test_quantization_error_is_small_vs_fp16(pkg, cuda, K, N):
    """Per-channel int8 on roughly Gaussian weights lands near 1% relative
    error; the reference's bound is 3%."""
    lin = _linear(K, N, False, cuda)
    q = pkg.QuantizedLinearInt8.from_linear(lin)
    x = _x(64, K, F16, cuda, seed=2)
    fp16_out = lin(x).float()
    int8_out = q(x).float()
    rel_err = ((fp16_out - int8_out).norm() / fp16_out.norm()).item()
    print(f"quantisation rel err [{K}->{N}]: {rel_err:.4f}")
    assert rel_err < 0.03


def test_roundtrip_error_within_half_a_quantization_step(pkg, cuda):
    lin = _linear(1536, 1536, False, cuda)
    q = pkg.QuantizedLinearInt8.from_linear(lin)
    original = lin.weight.float()
    dequantized = q.dequantized_weight(torch.float32)
    max_allowed = (q.scale[:, None] / 2) * 1.001 + 1e-6
    assert ((original - dequantized).abs() <= max_allowed).all()


def test_weight_bytes_roughly_halved(pkg, cuda):
    lin = _linear(1536, 8960, False, cuda)
    q = pkg.QuantizedLinearInt8.from_linear(lin)
    fp16_bytes = lin.weight.numel() * lin.weight.element_size()
    assert q.num_bytes() < 0.55 * fp16_bytes


@pytest.mark.parametrize("wdt", [F32, BF16])
def test_quantizer_other_weight_dtypes_and_special_rows(pkg, orc, cuda, wdt):
    N, K = 40, 300
    w = torch.randn(N, K, generator=gen(8)) * 0.05
    w[0] = 0.0                                           # scale floor 1e-8
    w[1] = 1e-12                                         # below the floor after / 127
    w[2, :8] = torch.tensor([127.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5, 1.5])   # scale 1: ties to even
    w[2, 8:] = 0.0
    w = w.to(wdt)
    q, s = pkg.quantize_int8_weight(w.to(cuda))
    oq, os_ = orc.quantize_int8(storage(w), wdt=DT_NAME[wdt])
    assert np.array_equal(q.cpu().numpy(), oq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), os_.view(np.uint32))
    if wdt == F32:
        assert q[2, :8].tolist() == [127, 2, -2, 4, -4, 0, 0, 2]


def test_quantizer_row_strided_weight(pkg, orc, cuda):
    big = torch.randn(48, 1600, generator=gen(12)).to(F16).to(cuda)
    view = big[:, 40:40 + 1536]
    q, s = pkg.quantize_int8_weight(view)
    q2, s2 = pkg.quantize_int8_weight(view.contiguous())
    assert torch.equal(q, q2) and torch.equal(s, s2)


def test_tiled_launch_shapes_agree_bitwise(pkg, cuda):
    """Every tiled shape (160 .. 4096 rows, n = 3584: 64 x 64 and 128 x 128
    on the step pipeline, 128 x 64, 256 x 128 and 256 x 256 on the sub-step
    ring) adds the k products in the same order: row prefixes of one input
    give the same bits whichever shape runs."""
    K, N = 1024, 3584
    lin = _linear(K, N, True, cuda, dtype=F16, seed=41)
    q = pkg.QuantizedLinearInt8.from_linear(lin)
    x = _x(4096, K, F16, cuda, seed=42)
    full = pkg.w8a16_linear(x, q.weight_q, q.scale, q.bias, out_dtype=F32)
    for r in (160, 600, 1200, 2048):
        part = pkg.w8a16_linear(x[:r], q.weight_q, q.scale, q.bias, out_dtype=F32)
        assert torch.equal(part, full[:r]), f"{r} rows differ from the 4096-row launch"


def test_strided_views_give_identical_bits(pkg, cuda):
    M, K, N = 12, 1536, 896
    lin = _linear(K, N, True, cuda, seed=3)
    q = pkg.QuantizedLinearInt8.from_linear(lin)
    x = _x(M, K, F16, cuda, seed=3)
    want = pkg.w8a16_linear(x, q.weight_q, q.scale, q.bias)
    xbig = torch.zeros((M, K + 24), dtype=F16, device=cuda)
    xbig[:, 8:8 + K] = x                       # row stride K + 24, base offset 16 bytes
    qbig = torch.zeros((N, K + 64), dtype=torch.int8, device=cuda)
    qbig[:, 16:16 + K] = q.weight_q
    got = pkg.w8a16_linear(xbig[:, 8:8 + K], qbig[:, 16:16 + K], q.scale, q.bias)
    assert torch.equal(got, want)
    assert torch.equal(pkg.w8a16_linear(x, q.weight_q, q.scale, q.bias), want)   # run to run


@pytest.mark.parametrize("M", [3, 40])
def test_misaligned_and_odd_k_take_the_generic_kernel(pkg, orc, cuda, M):
    """x at a 2-byte offset, and k = 1000 (not a multiple of 16): same
    contract, served by the generic kernel."""
    K, N = 1000, 64
    lin = _linear(K, N, True, cuda, seed=6)
    q = pkg.QuantizedLinearInt8.from_linear(lin)
    xbig = _x(M, K + 1, F16, cuda, seed=9)
    x = xbig[:, 1:]                             # row stride K + 1, 2-byte misaligned
    got16 = pkg.w8a16_linear(x, q.weight_q, q.scale, q.bias)
    got32 = pkg.w8a16_linear(x, q.weight_q, q.scale, q.bias, out_dtype=F32)
    _check_kernel(orc, x.contiguous(), q, got16, got32)
    K2 = 1024
    lin2 = _linear(K2, N, False, cuda, seed=10)
    q2 = pkg.QuantizedLinearInt8.from_linear(lin2)
    x2 = _x(M, K2 + 1, F16, cuda, seed=11)[:, 1:]
    _check_kernel(orc, x2.contiguous(), q2, pkg.w8a16_linear(x2, q2.weight_q, q2.scale),
                  pkg.w8a16_linear(x2, q2.weight_q, q2.scale, out_dtype=F32))


@pytest.mark.parametrize("M", [5, 13])
def test_out_row_stride_through_abi(pkg, cuda, M):
    L = importlib.import_module("llm-inference-optimizer_amd._lib")
    K, N = 256, 48
    lin = _linear(K, N, True, cuda, dtype=BF16, seed=13)
    q = pkg.QuantizedLinearInt8.from_linear(lin)
    x = _x(M, K, BF16, cuda, seed=14)
    want = pkg.w8a16_linear(x, q.weight_q, q.scale, q.bias)
    out = torch.full((M, N + 5), 7.0, dtype=BF16, device=cuda)
    L.w8a16_linear_fwd(x.data_ptr(), q.weight_q.data_ptr(), q.scale.data_ptr(), q.bias.data_ptr(), out.data_ptr(),
                       M, K, N, K, K, N + 5, L.BF16, L.F32, L.BF16, L.BF16, L.stream_handle(cuda))
    torch.cuda.synchronize()
    assert torch.equal(out[:, :N], want)
    assert torch.all(out[:, N:] == 7.0)


@pytest.mark.parametrize("M,K,N", [(8, 1536, 8960), (16, 1536, 8960), (100, 1536, 8960),
                                   # 17 - 64 rows on the stream kernel (6, 8, 12 and 16 x sets)
                                   (32, 8960, 1536), (20, 4864, 896), (44, 8960, 1536), (64, 4864, 896),
                                   # the 16-row class balanced over the CUs
                                   (8, 13824, 5120)])
def test_graph_replays_match_eager(pkg, cuda, M, K, N):
    lin = _linear(K, N, False, cuda, seed=15)
    q = pkg.QuantizedLinearInt8.from_linear(lin)
    x = _x(M, K, F16, cuda, seed=16)
    xs = x.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        q(xs)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = q(xs)
    for i in range(4):
        xs.copy_(x * (1 + 0.25 * i))
        graph.replay()
        torch.cuda.synchronize()
        want = q(xs)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i} differs from eager"


@pytest.mark.parametrize("M,K,N", [(8, 3584, 18944), (32, 18944, 3584), (512, 3584, 4608),
                                   # the sub-step ring's 256 x 128 and 256 x 256 tiles with a main loop
                                   (2048, 3584, 3584), (4096, 1024, 3584)])
def test_qwen7b_shapes_against_fp64(pkg, orc, cuda, M, K, N):
    lin = _linear(K, N, False, cuda, dtype=BF16, seed=17)
    q = pkg.QuantizedLinearInt8.from_linear(lin)
    x = _x(M, K, BF16, cuda, seed=18)
    got16 = pkg.w8a16_linear(x, q.weight_q, q.scale)
    got32 = pkg.w8a16_linear(x, q.weight_q, q.scale, out_dtype=F32)
    same = _check_kernel(orc, x, q, got16, got32, max_oracle_macs=1e7)
    print(f"7B-shape W8A16 [{M}x{K}] x [{N}x{K}]: {same:.5f} equal to the oracle")
