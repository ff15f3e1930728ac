"""GPU checks of the 16-bit linear (``mi355_linear16_fwd``), which FusedMLP's
down projection (src/engine/fused_norm_activation_patch.py:64) runs with
``hip_down=True``:

* parity with the oracle (``oracle.linear16``) over the down / q / k / o
  projection shapes of Qwen2.5-0.5B/1.5B/7B at decode rows, K tails, ragged
  feature counts, > 32 rows (the tiled GEMM), bias in
  three dtypes, fp16 and bf16.  The kernels sum in fp32 in their own order,
  so the bar is the exact value within one output ulp plus the worst-case
  fp32 summation error gamma_k * sum |x * w|; on top of that >= 99% of
  outputs must equal the oracle's single rounding bit for bit, the fp32
  output must sit within the bound, and the 16-bit output must be the fp32
  output rounded once;
* torch's own linear (hipBLASLt) on the same inputs agrees within both
  sides' bounds, equals this kernel on >= 95% of outputs, and is no closer
  to the exact value on average;
* odd k and misaligned views (the generic kernel), strided views, 3-D
  inputs, determinism, graph replay, prefill shapes against fp64 GEMMs on
  the GPU, and the FusedMLP ``hip_down`` path in a patched model.
"""
import importlib

import numpy as np
import pytest
import torch

from parity_utils import DT_NAME, randn, storage, ulp16

pytestmark = pytest.mark.gpu

F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32


def _inputs(rows, k, n, dt, seed, bias_dt=None):
    x = randn((rows, k), seed, dt)
    w = randn((n, k), seed + 1, dt, std=k ** -0.5)
    b = None if bias_dt is None else randn((n,), seed + 2, bias_dt, std=0.5)
    return x, w, b


def _gamma(k):
    return k * 2.0 ** -24 / (1 - k * 2.0 ** -24)


def _check_vs_oracle(orc, got16, got32, x, w, b, dt):
    name = DT_NAME[dt]
    k = x.shape[1]
    r = orc.linear16(storage(x), storage(w), None if b is None else storage(b), dt=name,
                     bdt=None if b is None else DT_NAME[b.dtype])
    exact = r["out64"]
    bound = _gamma(k) * r["absacc"] + 2.0 ** -24 * np.abs(exact)  # sums, then the fp32 bias add
    g16 = orc.to_f32(storage(got16), name).astype(np.float64)
    err16 = np.abs(g16 - exact)
    tol16 = ulp16(exact, dt) + bound
    assert np.all(err16 <= tol16), f"max excess {np.max(err16 - tol16):.3e}"
    same = float(np.mean(storage(got16) == r["out"]))
    assert same >= 0.99, f"only {same:.4f} of outputs equal the single-rounding oracle"
    e32 = np.abs(got32.numpy().astype(np.float64) - exact)
    assert np.all(e32 <= bound + 1e-30), f"fp32 excess {np.max(e32 - bound):.3e}"
    assert torch.equal(got16, got32.to(dt)), "the 16-bit output is not the fp32 output rounded once"
    return same, float(np.max(err16 / ulp16(exact, dt)))


@pytest.mark.parametrize("rows,k,n,dt,bias", [
    # decode rows: the weight-streaming kernel (down, q/o, k/v, 7B down, 0.5B down)
    (1, 8960, 1536, F16, None), (8, 8960, 1536, F16, None), (4, 8960, 1536, BF16, "f32"),
    (32, 8960, 1536, F16, "same"), (16, 1536, 1536, BF16, "same"), (2, 1536, 256, F16, "f16"),
    (8, 18944, 3584, BF16, None), (3, 4864, 896, BF16, None), (24, 3584, 3584, F16, None),
    (12, 18944, 3584, BF16, "f32"), (16, 8960, 1536, F16, "same"), (13, 3104, 2900, F16, None),
    (1, 136, 1000, BF16, "f16"), (6, 3584, 18944, F16, None),
    # 4 rows on deep rows of outputs that are not narrow: 16-row workgroups
    # (a partial last chunk and a ragged last workgroup at k 3104 x n 4204)
    (4, 3104, 4204, BF16, "f32"), (4, 18944, 3584, F16, None),
    (17, 4864, 896, BF16, "f32"), (29, 3104, 2900, F16, None), (32, 18944, 3584, BF16, "same"),
    (57, 3104, 2900, F16, "f32"), (64, 4864, 896, BF16, None), (40, 1552, 37, F16, "same"),
    # k tails (not a multiple of 64), ragged n, tiny shapes
    (5, 72, 40, F16, "f32"), (7, 8, 3, BF16, None), (9, 1000, 77, F16, "same"), (1, 8, 1, F16, None),
    # more than 32 rows: the tiled GEMM (k tails, ragged edges, small grids)
    (33, 1536, 256, F16, None), (100, 256, 100, BF16, "same"), (200, 8960, 1536, F16, "f32"),
    (300, 1552, 520, BF16, None), (257, 96, 333, F16, "same"),
    # the small tiled shapes: >= 128 tile columns at 17 - 32 rows, any 33 - 64 rows
    (24, 512, 8192, F16, "f32"), (20, 256, 16400, BF16, None), (48, 8960, 1536, F16, "same"),
    (64, 1000, 200, BF16, None),
])
def test_linear16_matches_oracle(pkg, orc, cuda, rows, k, n, dt, bias):
    bias_dt = None if bias is None else (dt if bias == "same" else {"f32": F32, "f16": F16}[bias])
    x, w, b = _inputs(rows, k, n, dt, seed=40 + rows + k, bias_dt=bias_dt)
    xd, wd = x.to(cuda), w.to(cuda)
    bd = None if b is None else b.to(cuda)
    got16 = pkg.linear16(xd, wd, bd).cpu()
    got32 = pkg.linear16(xd, wd, bd, out_dtype=F32).cpu()
    assert got16.shape == (rows, n) and got16.dtype == dt
    same, mx = _check_vs_oracle(orc, got16, got32, x, w, b, dt)
    print(f"linear16 [{rows}x{k}] x [{n}x{k}] {dt} bias={bias}: {same:.5f} equal to oracle, max err {mx:.2f} ulp")


@pytest.mark.parametrize("rows,dt", [(1, F16), (8, BF16), (32, F16)])
def test_linear16_agrees_with_torch_linear(pkg, cuda, rows, dt):
    """Against torch's own linear (hipBLASLt) on the same inputs and the exact
    (fp64) value: both sum in fp32 in different orders (and torch may add the
    bias after rounding), so they may differ by an ulp or two on a few
    outputs; this kernel's outputs are at least as close to exact."""
    k, n = 8960, 1536
    x, w, b = (t.to(cuda) for t in _inputs(rows, k, n, dt, seed=3, bias_dt=dt))
    got = pkg.linear16(x, w, b).double()
    want = torch.nn.functional.linear(x, w, b).double()
    exact = x.double() @ w.double().T + b.double()
    ulp = torch.from_numpy(ulp16(exact.cpu().numpy(), dt)).to(cuda)
    # each side: one output ulp plus any fp32 summation order's error (gamma_k sum |x w|)
    bound = _gamma(k) * (x.double().abs() @ w.double().abs().T) + 2.0 ** -24 * exact.abs()
    assert float(((got - want).abs() - 2 * (ulp + bound)).max()) <= 0, "further from torch's linear than two bounds"
    frac = float((got != want).double().mean())
    e_ours, e_torch = float((got - exact).abs().mean()), float((want - exact).abs().mean())
    print(f"linear16 vs torch linear, {rows} rows {dt}: {frac:.4f} of outputs differ; "
          f"mean |err| {e_ours:.3e} (this kernel) vs {e_torch:.3e} (torch)")
    assert frac < 0.05
    assert e_ours <= 1.02 * e_torch


def test_generic_kernel_odd_k_and_misaligned_views(pkg, orc, cuda):
    """k not a multiple of 8 and an x view 2 bytes off 16-byte alignment take
    the generic kernel: same bar against the oracle."""
    for rows, k, n, off in ((6, 61, 35, 0), (9, 1536, 96, 1)):
        x, w, b = _inputs(rows, k, n, F16, seed=7 + k, bias_dt=F16)
        xbig = torch.zeros((rows, k + 8), dtype=F16)
        xbig[:, off:off + k] = x
        xd = xbig.to(cuda)[:, off:off + k]
        got16 = pkg.linear16(xd, w.to(cuda), b.to(cuda)).cpu()
        got32 = pkg.linear16(xd, w.to(cuda), b.to(cuda), out_dtype=F32).cpu()
        _check_vs_oracle(orc, got16, got32, x, w, b, F16)


def test_strided_views_and_3d_input_give_identical_bits(pkg, cuda):
    rows, k, n = 12, 8960, 1536
    x, w, _ = (None if t is None else t.to(cuda) for t in _inputs(rows, k, n, BF16, seed=5))
    want = pkg.linear16(x, w)
    xbig = torch.zeros((rows, k + 24), dtype=BF16, device=cuda)
    xbig[:, 8:8 + k] = x                      # row stride k + 24, base offset 16 bytes
    wbig = torch.zeros((n, k + 64), dtype=BF16, device=cuda)
    wbig[:, :k] = w
    assert torch.equal(pkg.linear16(xbig[:, 8:8 + k], wbig[:, :k]), want)
    got3 = pkg.linear16(x.view(3, 4, k), w)
    assert got3.shape == (3, 4, n) and torch.equal(got3.view(rows, n), want)
    assert torch.equal(pkg.linear16(x, w), want)   # run to run


def test_out_row_stride_through_abi(pkg, cuda):
    """Writing into a row-strided output leaves the gaps untouched."""
    L = importlib.import_module("llm-inference-optimizer_amd._lib")
    rows, k, n = 5, 1536, 48
    x, w, b = (t.to(cuda) for t in _inputs(rows, k, n, F16, seed=9, bias_dt=F16))
    want = pkg.linear16(x, w, b)
    out = torch.full((rows, n + 5), 7.0, dtype=F16, device=cuda)
    L.linear16_fwd(x.data_ptr(), w.data_ptr(), b.data_ptr(), out.data_ptr(), rows, k, n, k, k, n + 5,
                   L.F16, L.F16, L.F16, L.stream_handle(cuda))
    torch.cuda.synchronize()
    assert torch.equal(out[:, :n], want)
    assert torch.all(out[:, n:] == 7.0)


def test_abi_rejects_bad_arguments(pkg, cuda):
    L = importlib.import_module("llm-inference-optimizer_amd._lib")
    x = torch.randn(4, 64, dtype=F16, device=cuda)
    w = torch.randn(16, 64, dtype=F16, device=cuda)
    out = torch.empty(4, 16, dtype=F16, device=cuda)
    s = L.stream_handle(cuda)
    with pytest.raises(L.KernelError, match="fp16 or bf16"):
        L.linear16_fwd(x.data_ptr(), w.data_ptr(), None, out.data_ptr(), 4, 64, 16, 64, 64, 16, L.F32, 0, L.F32, s)
    with pytest.raises(L.KernelError, match="row strides"):
        L.linear16_fwd(x.data_ptr(), w.data_ptr(), None, out.data_ptr(), 4, 64, 16, 32, 64, 16, L.F16, 0, L.F16, s)
    with pytest.raises(L.KernelError, match="out dtype"):
        L.linear16_fwd(x.data_ptr(), w.data_ptr(), None, out.data_ptr(), 4, 64, 16, 64, 64, 16, L.F16, 0, L.BF16, s)
    with pytest.raises(AssertionError, match="dtype mismatch"):
        pkg.linear16(x, w.to(BF16))


@pytest.mark.parametrize("rows,k,n", [(8, 8960, 1536), (32, 8960, 1536), (13, 18944, 3584), (64, 8960, 1536)])
def test_graph_replays_match_eager(pkg, cuda, rows, k, n):
    x, w, b = (t.to(cuda) for t in _inputs(rows, k, n, F16, seed=11, bias_dt=F32))
    xs = x.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pkg.linear16(xs, w, b)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = pkg.linear16(xs, w, b)
    for i in range(4):
        xs.copy_(x * (1 + 0.25 * i))
        graph.replay()
        torch.cuda.synchronize()
        want = pkg.linear16(xs, w, b)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i} differs from eager"


@pytest.mark.parametrize("rows,k,n,dt", [(1024, 8960, 1536, F16), (2048, 3584, 4736, BF16)])
def test_prefill_shapes_against_torch_fp64(pkg, cuda, rows, k, n, dt):
    """Prefill-sized batches (the tiled GEMM) against fp64 GEMMs on the GPU:
    every output within one output ulp plus the fp32 summation bound, the
    fp32 output within the bound, the 16-bit output the fp32 one rounded once."""
    torch.manual_seed(rows)
    x = torch.randn(rows, k, device=cuda).to(dt)
    w = (torch.randn(n, k, device=cuda) * k ** -0.5).to(dt)
    b = torch.randn(n, device=cuda).to(dt)
    got16 = pkg.linear16(x, w, b).double()
    got32 = pkg.linear16(x, w, b, out_dtype=F32).double()
    exact = x.double() @ w.double().T + b.double()
    bound = _gamma(k) * (x.double().abs() @ w.double().abs().T) + 2.0 ** -24 * exact.abs()
    ulp = torch.from_numpy(ulp16(exact.cpu().numpy(), dt)).to(cuda)
    assert float(((got32 - exact).abs() - bound).max()) <= 1e-30
    assert float(((got16 - exact).abs() - (ulp + bound)).max()) <= 0
    assert torch.equal(got16.to(dt), got32.to(dt))


def test_fused_mlp_hip_down_takes_the_kernel_for_decode_rows(pkg, cuda, monkeypatch):
    pytest.importorskip("transformers")
    from transformers import Qwen2Config, Qwen2ForCausalLM
    patch_mod = importlib.import_module("llm-inference-optimizer_amd.engine.fused_norm_activation_patch")
    cfg = Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=1024, num_hidden_layers=4,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=128)
    torch.manual_seed(0)
    base = Qwen2ForCausalLM(cfg).to(device=cuda, dtype=F16).eval()
    fused = Qwen2ForCausalLM(cfg).to(device=cuda, dtype=F16).eval()
    fused.load_state_dict(base.state_dict())
    counts = pkg.patch_model_with_fused_kernels(fused, fuse_gate_up=True, hip_down=True)
    assert counts == {"rmsnorm": 9, "mlp": 4, "gate_up": 4, "down": 4}
    calls = []
    real = patch_mod.linear16

    def counting(*a, **kw):
        calls.append(tuple(a[0].shape))
        return real(*a, **kw)

    monkeypatch.setattr(patch_mod, "linear16", counting)
    ids = torch.randint(0, 512, (2, 40), device=cuda)
    with torch.inference_mode():
        lb = base(ids[:, :8]).logits.float()       # 16 rows: the HIP down projection
        lf = fused(ids[:, :8]).logits.float()
        assert len(calls) == 4
        pb = base(ids).logits.float()              # 80 rows: torch's linear
        pf = fused(ids).logits.float()
        assert len(calls) == 4
    for a, b in ((lb, lf), (pb, pf)):
        err = (a - b).abs().max().item()
        assert err <= 0.05 * a.abs().max().item(), err
