"""GPU checks of the fused gate/up projections + SiLU-and-mul
(``mi355_gate_up_silu_fwd``; the fusion the reference's design lists next,
docs/architecture-cuda.md:94, of the MLP its FusedMLP runs as two GEMMs and
``fused_silu_mul``, src/engine/fused_norm_activation_patch.py:60-64):

* parity with the oracle (``oracle.gate_up_silu``) over decode shapes of
  Qwen2.5-0.5B/1.5B/7B, K tails, ragged feature counts and > 32 rows.  The
  kernel accumulates in fp32 in its own order, so the bar is the exact value
  within one output ulp plus the worst-case fp32 summation error
  (gamma_k = k * 2^-24 of sum |x * w|) carried through the activation; on
  top of that >= 99% of outputs must equal the oracle's single-rounding
  result bit for bit, and the fp32 output must sit within that bound too;
* the fused result is closer to the exact value than the reference's
  unfused chain (GEMMs rounded to x's type, then fused_silu_mul);
* strides, 3-D inputs, determinism, graph replay, the FusedMLP opt-in path
  and a 70B-class shape against a torch fp64 reference on the GPU.
"""
import importlib

import numpy as np
import pytest
import torch

from parity_utils import DT_NAME, randn, storage

pytestmark = pytest.mark.gpu

F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32


def _inputs(rows, k, n, dt, seed):
    x = randn((rows, k), seed, dt)
    wg = randn((n, k), seed + 1, dt, std=2.0 * k ** -0.5)
    wu = randn((n, k), seed + 2, dt, std=k ** -0.5)
    return x, wg, wu


def _ulp(v: np.ndarray, dt) -> np.ndarray:
    mant, emin = (10, -14) if dt == F16 else (7, -126)
    e = np.maximum(np.floor(np.log2(np.maximum(np.abs(v), 1e-300))), emin)
    return 2.0 ** (e - mant)


def _act_error_bound(g, u, gabs, uabs, k):
    """Worst-case effect of fp32 summation (any order) of the projections on
    silu(g) * u: gamma_k * sum|x w| per projection, through the derivatives."""
    gam = k * 2.0 ** -24 / (1 - k * 2.0 ** -24)
    eg, eu = gam * gabs, gam * uabs
    sig = 1.0 / (1.0 + np.exp(-g))
    dsilu = sig * (1.0 + g * (1.0 - sig))
    # second-order slack: |silu''| <= 0.5
    return np.abs(dsilu * u) * eg + np.abs(g * sig) * eu + eg * eu + 0.5 * eg * eg * np.abs(u)


def _check_vs_oracle(orc, got16, got32, x, wg, wu, dt):
    name = DT_NAME[dt]
    k = x.shape[1]
    r = orc.gate_up_silu(storage(x), storage(wg), storage(wu), dt=name)
    exact = r["out64"]
    bound = _act_error_bound(r["g"], r["u"], r["gabs"], r["uabs"], k)
    g16 = orc.to_f32(storage(got16), name).astype(np.float64)
    err16 = np.abs(g16 - exact)
    tol16 = _ulp(exact, dt) + bound + 2.0 ** -22 * np.abs(exact)
    assert np.all(err16 <= tol16), f"max excess {np.max(err16 - tol16):.3e}"
    same = float(np.mean(storage(got16) == r["out"]))
    assert same >= 0.99, f"only {same:.4f} of outputs equal the single-rounding oracle"
    e32 = np.abs(got32.numpy().astype(np.float64) - exact)
    assert np.all(e32 <= 2.0 ** -22 * np.abs(exact) + bound + 1e-30), f"fp32 excess {np.max(e32 - bound):.3e}"
    return same, float(np.max(err16 / _ulp(exact, dt)))


@pytest.mark.parametrize("rows,k,n,dt", [
    (8, 1536, 8960, F16), (1, 1536, 8960, BF16), (32, 1536, 8960, F16), (16, 896, 4864, BF16),
    (4, 3584, 18944, BF16), (5, 72, 40, F16), (33, 40, 24, BF16), (3, 8, 7, F16), (100, 256, 100, BF16),
    # up to 8 rows: the weight-streaming kernel's three launch shapes, k tails past a 128-column chunk,
    # ragged weight-row counts
    (6, 3584, 1000, BF16), (7, 136, 520, F16), (2, 2056, 264, F16), (8, 2048, 4099, BF16), (1, 24, 1, F16),
    (12, 1536, 8960, F16), (13, 136, 1000, BF16), (16, 3584, 2000, F16), (9, 2056, 37, BF16),
    (11, 3104, 2900, BF16), (32, 896, 4864, BF16), (21, 3104, 2900, F16),
    (17, 2048, 1000, F16),
    # 9 - 16 rows: 4-row workgroups where 8-row ones would number under 4 per
    # CU (ragged last workgroup), 16-row ones of about 5 waves per CU from k = 2048
    (10, 896, 4874, F16), (12, 2048, 11008, BF16),
    # prefill rows: the tiled GEMM (each of its three launch shapes, k tails, ragged edges)
    (64, 1536, 1000, F16), (200, 640, 10240, BF16), (300, 1552, 520, F16), (257, 96, 333, BF16),
    # 17 - 64 rows: the small tiled shapes (32 x 64, 32 x 128 for n_out > 10000, 64 x 64)
    (20, 256, 16400, BF16), (24, 1536, 8960, F16), (40, 256, 4000, F16), (63, 136, 72, BF16),
    # > 128 rows, few tiles: 256 x 64 (main loop and k tail; tail only)
    (1100, 1000, 300, F16), (1030, 72, 130, BF16),
])
def test_gate_up_silu_matches_oracle(pkg, orc, cuda, rows, k, n, dt):
    x, wg, wu = _inputs(rows, k, n, dt, seed=80 + rows)
    xd, wgd, wud = x.to(cuda), wg.to(cuda), wu.to(cuda)
    got16 = pkg.fused_gate_up_silu(xd, wgd, wud).cpu()
    got32 = pkg.fused_gate_up_silu(xd, wgd, wud, out_dtype=F32).cpu()
    assert got16.shape == (rows, n) and got16.dtype == dt
    same, mx = _check_vs_oracle(orc, got16, got32, x, wg, wu, dt)
    print(f"gate_up_silu [{rows}x{k}] x [{n}x{k}] {dt}: {same:.5f} equal to oracle, max err {mx:.2f} ulp")


@pytest.mark.parametrize("dt", [F16, BF16])
def test_fused_is_closer_to_exact_than_the_unfused_chain(pkg, orc, cuda, dt):
    """The reference's FusedMLP computes fused_silu_mul(gate_proj(x),
    up_proj(x)) with both projections rounded to x's type; dropping that
    rounding moves the result toward the exact value."""
    rows, k, n = 8, 1536, 8960
    x, wg, wu = _inputs(rows, k, n, dt, seed=7)
    xd, wgd, wud = x.to(cuda), wg.to(cuda), wu.to(cuda)
    fused = pkg.fused_gate_up_silu(xd, wgd, wud).cpu()
    chain = pkg.fused_silu_mul(xd @ wgd.T, xd @ wud.T).cpu()
    exact = orc.gate_up_silu(storage(x), storage(wg), storage(wu), dt=DT_NAME[dt])["out64"]
    e_fused = np.abs(fused.double().numpy() - exact).mean()
    e_chain = np.abs(chain.double().numpy() - exact).mean()
    print(f"{dt}: mean |err| fused {e_fused:.3e}, unfused chain {e_chain:.3e}")
    assert e_fused < e_chain


def test_strided_views_and_3d_input_give_identical_bits(pkg, cuda):
    rows, k, n = 12, 1536, 896
    x, wg, wu = (t.to(cuda) for t in _inputs(rows, k, n, F16, seed=3))
    want = pkg.fused_gate_up_silu(x, wg, wu)
    xbig = torch.zeros((rows, k + 24), dtype=F16, device=cuda)
    xbig[:, 8:8 + k] = x                      # row stride k + 24, base offset 16 bytes
    wgbig = torch.zeros((n, k + 64), dtype=F16, device=cuda)
    wubig = torch.zeros((n, k + 64), dtype=F16, device=cuda)
    wgbig[:, :k] = wg
    wubig[:, :k] = wu
    got = pkg.fused_gate_up_silu(xbig[:, 8:8 + k], wgbig[:, :k], wubig[:, :k])
    assert torch.equal(got, want)
    got3 = pkg.fused_gate_up_silu(x.view(3, 4, k), wg, wu)
    assert got3.shape == (3, 4, n) and torch.equal(got3.view(rows, n), want)
    assert torch.equal(pkg.fused_gate_up_silu(x, wg, wu), want)   # run to run


@pytest.mark.parametrize("rows,k,n", [(5, 256, 48), (1024, 64, 8960)])  # decode rows; a column split
def test_out_row_stride_through_abi(pkg, cuda, rows, k, n):
    """Writing into a row-strided output leaves the gaps untouched."""
    L = importlib.import_module("llm-inference-optimizer_amd._lib")
    x, wg, wu = (t.to(cuda) for t in _inputs(rows, k, n, BF16, seed=9))
    want = pkg.fused_gate_up_silu(x, wg, wu)
    out = torch.full((rows, n + 5), 7.0, dtype=BF16, device=cuda)
    L.gate_up_silu_fwd(x.data_ptr(), wg.data_ptr(), wu.data_ptr(), out.data_ptr(), rows, k, n, k, k, n + 5,
                       L.BF16, L.BF16, L.stream_handle(cuda))
    torch.cuda.synchronize()
    assert torch.equal(out[:, :n], want)
    assert torch.all(out[:, n:] == 7.0)


@pytest.mark.parametrize("rows", [40, 8])
def test_huge_x_row_stride(pkg, orc, cuda, rows):
    """An x row stride of 2^22 + 8 elements is past what the tiled GEMM's
    buffer descriptors span: 40 rows then run the skinny weight-streaming
    kernel (the stream kernel serves up to 32 rows), 8 rows the stream
    kernel, whose x descriptor still spans them; both against the oracle."""
    L = importlib.import_module("llm-inference-optimizer_amd._lib")
    k, n, xs = 256, 300, (1 << 22) + 8
    x, wg, wu = _inputs(rows, k, n, F16, seed=77)
    xbig = torch.zeros((rows, xs), dtype=F16, device=cuda)
    xbig[:, :k] = x.to(cuda)
    wgd, wud = wg.to(cuda), wu.to(cuda)
    out16 = torch.empty((rows, n), dtype=F16, device=cuda)
    out32 = torch.empty((rows, n), dtype=F32, device=cuda)
    for out, odt in ((out16, L.F16), (out32, L.F32)):
        L.gate_up_silu_fwd(xbig.data_ptr(), wgd.data_ptr(), wud.data_ptr(), out.data_ptr(), rows, k, n, xs, k, n,
                           L.F16, odt, L.stream_handle(cuda))
    torch.cuda.synchronize()
    _check_vs_oracle(orc, out16.cpu(), out32.cpu(), x, wg, wu, F16)


def test_misaligned_k_is_rejected(pkg, cuda):
    L = importlib.import_module("llm-inference-optimizer_amd._lib")
    x = torch.randn(4, 60, dtype=F16, device=cuda)
    w = torch.randn(16, 60, dtype=F16, device=cuda)
    with pytest.raises(L.KernelError, match="multiples of 8"):
        pkg.fused_gate_up_silu(x, w, w)


@pytest.mark.parametrize("rows,k,n", [(8, 1536, 8960), (16, 1536, 8960), (32, 896, 4864)])
def test_graph_replays_match_eager(pkg, cuda, rows, k, n):
    x, wg, wu = (t.to(cuda) for t in _inputs(rows, k, n, BF16, seed=11))
    xs = x.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pkg.fused_gate_up_silu(xs, wg, wu)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = pkg.fused_gate_up_silu(xs, wg, wu)
    for i in range(4):
        xs.copy_(x * (1 + 0.25 * i))
        graph.replay()
        torch.cuda.synchronize()
        want = pkg.fused_gate_up_silu(xs, wg, wu)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i} differs from eager"


def test_large_shape_against_torch_fp64(pkg, cuda):
    """32 decode rows against 28672 x 8192 weights (a 70B-class MLP, 940 MB of
    weights): the exact value from fp64 GEMMs on the GPU."""
    rows, k, n = 32, 8192, 28672
    torch.manual_seed(0)
    x = torch.randn(rows, k, device=cuda).to(BF16)
    wg = (torch.randn(n, k, device=cuda) * (2.0 * k ** -0.5)).to(BF16)
    wu = (torch.randn(n, k, device=cuda) * k ** -0.5).to(BF16)
    got = pkg.fused_gate_up_silu(x, wg, wu, out_dtype=F32).double()
    x64 = x.double()
    g, u = x64 @ wg.double().T, x64 @ wu.double().T
    gabs, uabs = x64.abs() @ wg.double().abs().T, x64.abs() @ wu.double().abs().T
    exact = torch.nn.functional.silu(g) * u
    bound = torch.from_numpy(_act_error_bound(g.cpu().numpy(), u.cpu().numpy(), gabs.cpu().numpy(),
                                              uabs.cpu().numpy(), k)).to(cuda)
    excess = (got - exact).abs() - (2.0 ** -22 * exact.abs() + bound)
    assert float(excess.max()) <= 1e-30
    rel = float(((got - exact).abs() / exact.abs().clamp_min(1e-3)).median())
    print(f"70B-class gate_up: median rel err {rel:.2e}")
    assert rel < 1e-5


@pytest.mark.parametrize("rows,k,n,dt", [
    (1024, 1536, 8960, F16), (2048, 3584, 4736, BF16),
    # ragged rows, k and n on the sub-step ring: 128 x 64 tiles two per CU,
    # then 256 x 128 tiles, then a column split (6528 columns in 256 x 128
    # tiles, the last 72 in 64 x 64)
    (300, 264, 8200, BF16), (520, 264, 8000, F16), (1030, 264, 6600, F16),
    # whole rounds that end inside a 128-column block: 768 tiles of 256 x 128
    # over 16384 columns (6 row blocks), then 2560 columns of 128 x 64 tiles
    (1536, 264, 18944, BF16),
])
def test_prefill_shapes_against_torch_fp64(pkg, cuda, rows, k, n, dt):
    """Prefill-sized batches (the tiled GEMM path) against fp64 GEMMs on the
    GPU: every output within one output ulp plus the fp32 summation bound,
    the fp32 output within the bound."""
    torch.manual_seed(rows)
    x = torch.randn(rows, k, device=cuda).to(dt)
    wg = (torch.randn(n, k, device=cuda) * (2.0 * k ** -0.5)).to(dt)
    wu = (torch.randn(n, k, device=cuda) * k ** -0.5).to(dt)
    got16 = pkg.fused_gate_up_silu(x, wg, wu).double()
    got32 = pkg.fused_gate_up_silu(x, wg, wu, out_dtype=F32).double()
    x64 = x.double()
    g, u = x64 @ wg.double().T, x64 @ wu.double().T
    gabs, uabs = x64.abs() @ wg.double().abs().T, x64.abs() @ wu.double().abs().T
    exact = torch.nn.functional.silu(g) * u
    bound = torch.from_numpy(_act_error_bound(g.cpu().numpy(), u.cpu().numpy(), gabs.cpu().numpy(),
                                              uabs.cpu().numpy(), k)).to(cuda)
    ulp = torch.from_numpy(_ulp(exact.cpu().numpy(), dt)).to(cuda)
    assert float(((got32 - exact).abs() - (2.0 ** -22 * exact.abs() + bound)).max()) <= 1e-30
    assert float(((got16 - exact).abs() - (ulp + bound + 2.0 ** -22 * exact.abs())).max()) <= 0
    # the 16-bit output is the fp32 output rounded once
    assert torch.equal(got16.to(dt), got32.to(dt))


def test_tiled_launch_shapes_agree_bitwise(pkg, cuda):
    """Every tiled launch shape (33 .. 1536 rows of the 1.5B MLP: 64 x 64,
    128 x 64 on 4 stages and on the sub-step ring, 256 x 64, 256 x 128 on the
    ring, and the column splits at 1024 and 1025 rows) adds the k products in
    the same order, so a prefix of the rows gives the same bits whichever
    shape runs."""
    torch.manual_seed(5)
    k, n = 1536, 8960
    x = torch.randn(1536, k, device=cuda).to(F16)
    wg = (torch.randn(n, k, device=cuda) * (2.0 * k ** -0.5)).to(F16)
    wu = (torch.randn(n, k, device=cuda) * k ** -0.5).to(F16)
    full = pkg.fused_gate_up_silu(x, wg, wu, out_dtype=F32)
    for rows in (33, 64, 65, 256, 257, 1024, 1025):
        part = pkg.fused_gate_up_silu(x[:rows], wg, wu, out_dtype=F32)
        assert torch.equal(part, full[:rows]), f"{rows} rows differ from the 1536-row launch"


def test_fused_mlp_opt_in_takes_the_fused_kernel(pkg, cuda, monkeypatch):
    transformers = pytest.importorskip("transformers")
    from transformers import Qwen2Config, Qwen2ForCausalLM
    patch_mod = importlib.import_module("llm-inference-optimizer_amd.engine.fused_norm_activation_patch")
    cfg = Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=1024, num_hidden_layers=4,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=128)
    torch.manual_seed(0)
    base = Qwen2ForCausalLM(cfg).to(device=cuda, dtype=BF16).eval()
    fused = Qwen2ForCausalLM(cfg).to(device=cuda, dtype=BF16).eval()
    fused.load_state_dict(base.state_dict())
    counts = pkg.patch_model_with_fused_kernels(fused, fuse_gate_up=True)
    assert counts == {"rmsnorm": 9, "mlp": 4, "gate_up": 4}
    calls = []
    real = patch_mod.fused_gate_up_silu

    def counting(*a, **kw):
        calls.append(a[0].shape)
        return real(*a, **kw)

    monkeypatch.setattr(patch_mod, "fused_gate_up_silu", counting)
    ids = torch.randint(0, 512, (2, 40), device=cuda)
    with torch.inference_mode():
        lb = base(ids[:, :8]).logits.float()       # 16 rows: fused projections (weight streaming)
        lf = fused(ids[:, :8]).logits.float()
        assert len(calls) == 4
        pb = base(ids).logits.float()              # 80 rows: fused projections (tiled GEMM)
        pf = fused(ids).logits.float()
        assert len(calls) == 8
    for a, b in ((lb, lf), (pb, pf)):
        err = (a - b).abs().max().item()
        assert err <= 0.05 * a.abs().max().item(), err
