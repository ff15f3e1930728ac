"""GPU checks of the int8 gate/up projections fused with SiLU-and-mul
(``mi355_gate_up_silu_w8a16_fwd``): the quantised MLP's two W8A16 linears
(src/quantization/int8.py:62-63) and its activation
(src/engine/fused_norm_activation_patch.py:60-64) as one kernel.

* parity with the oracle (``oracle.gate_up_silu_w8a16``, the composition of
  the pinned W8A16 and SiLU-and-mul oracles): every output within one output
  ulp plus the worst-case fp32 summation error of both projections carried
  through the activation; >= 99% of outputs equal to the oracle's
  single-rounding result; the fp32 output within the bound; the 16-bit output
  equal to the fp32 output rounded once -- over decode rows (the dual
  weight-streaming kernel), prefill rows (the dual tiled GEMM), odd k and
  misaligned inputs (the dual generic kernel), fp16 and bf16;
* the fused result is closer to the exact value than the reference's chain
  (two W8A16 linears rounded to x's dtype, then SiLU-and-mul);
* graph replay, a patched quantised model routing its MLPs through the
  kernel, and a prefill shape against fp64 GEMMs on the GPU.
"""
import importlib

import numpy as np
import pytest
import torch

from parity_utils import DT_NAME, act_error_bound, gen, storage, ulp16

pytestmark = pytest.mark.gpu

F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32


def _quantized(n, k, dt, seed, std, cuda, pkg):
    w = (torch.randn(n, k, generator=gen(seed)) * std).to(dt).to(cuda)
    return pkg.quantize_int8_weight(w)


def _inputs(rows, k, n, dt, seed, cuda, pkg):
    x = (torch.randn(rows, k, generator=gen(seed))).to(dt).to(cuda)
    qg, sg = _quantized(n, k, dt, seed + 1, 2.0 * k ** -0.5, cuda, pkg)
    qu, su = _quantized(n, k, dt, seed + 2, k ** -0.5, cuda, pkg)
    return x, qg, sg, qu, su


def _check(orc, x, qg, sg, qu, su, got16, got32):
    dt = x.dtype
    k = x.shape[1]
    r = orc.gate_up_silu_w8a16(storage(x), qg.cpu().numpy(), sg.cpu().numpy(), qu.cpu().numpy(),
                               su.cpu().numpy(), xdt=DT_NAME[dt])
    exact = r["out64"]
    bound = act_error_bound(r["g"], r["u"], r["gabs"], r["uabs"], k)
    g16 = got16.double().cpu().numpy()
    tol16 = ulp16(exact, dt) + bound + 2.0 ** -22 * np.abs(exact)
    assert np.all(np.abs(g16 - exact) <= tol16), f"max excess {np.max(np.abs(g16 - exact) - tol16):.3e}"
    e32 = np.abs(got32.double().cpu().numpy() - exact)
    assert np.all(e32 <= 2.0 ** -22 * np.abs(exact) + bound + 1e-30), "fp32 output outside the bound"
    same = float(np.mean(storage(got16.cpu()) == r["out"]))
    assert same >= 0.99, f"only {same:.4f} of outputs equal the oracle's single rounding"
    assert torch.equal(got16, got32.to(dt)), "the 16-bit output must be the fp32 output rounded once"
    return same


@pytest.mark.parametrize("rows,k,n,dt", [
    (1, 1536, 8960, F16), (8, 1536, 8960, F16), (8, 1536, 8960, BF16), (16, 896, 4864, BF16),
    (24, 1536, 1000, F16), (32, 2048, 512, F16), (4, 3584, 18944, BF16),
    # the 7B MLP at 1 and 8 rows
    (1, 3584, 18944, BF16), (8, 3584, 18944, BF16),
    # decode rows with a partial last 256-column chunk and a ragged last workgroup
    (3, 272, 1000, F16), (6, 1552, 520, BF16), (2, 4864, 904, F16),
    # 2 - 4 rows at k >= 3072 (8-row workgroups of 8 waves; a partial last
    # chunk and a ragged last workgroup at 3104 x 4204)
    (2, 3584, 18944, F16), (3, 3104, 4204, F16), (4, 3104, 4204, BF16),
    # 5 - 32 rows where 8-row workgroups would number under 4 per CU: 4-row
    # workgroups of 2 waves (ragged last workgroup)
    (6, 896, 4874, BF16), (12, 896, 4864, F16), (24, 1024, 3002, BF16),
    # 17 - 32 rows on 8-row workgroups of one wave: at 17 - 24 rows of MLPs
    # with k <= 2048 in place of the small tiles (ragged last workgroup), and
    # where the small tiles do not pay (3B MLP)
    (20, 1536, 8964, F16), (24, 2048, 11008, BF16), (30, 2048, 11008, F16),
    # 5 - 16 rows at k >= 3072 where the 16-row class numbers under 4
    # workgroups per CU: two waves (ragged last workgroup, partial last chunk)
    (6, 3104, 6004, F16), (12, 3104, 6004, BF16),
    # 2 - 4 rows below k = 3072: two chunks in flight per wave (a ragged last
    # workgroup; a partial last chunk and an odd chunk count at k 2064)
    (2, 1536, 8960, F16), (4, 896, 4874, BF16), (3, 2064, 11008, F16),
    # 33 - 48 rows where the small tiles do not pay: 12 x sets, one 4-row
    # weight set per workgroup, one wave (a ragged last workgroup)
    (40, 896, 4864, F16), (48, 896, 4874, BF16),
    # 9 - 16 rows: three and four x sets; the 7B MLP and k >= 3072 with n > 2048 (16-row
    # workgroups, one wave; a partial last chunk and a ragged last workgroup at k 3104 x n 2900)
    (12, 1536, 8960, F16), (13, 272, 1000, BF16), (16, 1552, 520, F16), (16, 3584, 18944, BF16),
    (12, 3584, 18944, BF16), (10, 3104, 2900, F16), (6, 3104, 2900, BF16), (15, 3104, 2900, BF16),
    # 17 - 32 rows where the small tiled shapes do not pay: the stream kernel with 6 and 8 x sets
    (20, 896, 4864, F16), (32, 3104, 2900, BF16), (25, 1552, 520, F16),
    # prefill rows: the dual tiled GEMM (and the skinny tiles of small grids)
    (33, 256, 100, BF16), (64, 1536, 1000, F16), (200, 640, 10240, F16), (300, 1552, 520, BF16),
    (1024, 1536, 2048, F16),
    # 17 - 64 rows with >= 128 tile columns: the small dual tiled shapes
    (32, 1536, 8960, F16), (20, 256, 16400, BF16), (56, 272, 8200, F16),
    # odd k: the dual generic kernel
    (5, 100, 37, F16), (40, 72, 40, BF16),
])
def test_matches_oracle(pkg, orc, cuda, rows, k, n, dt):
    x, qg, sg, qu, su = _inputs(rows, k, n, dt, 300 + rows, cuda, pkg)
    got16 = pkg.fused_gate_up_silu_w8a16(x, qg, sg, qu, su)
    got32 = pkg.fused_gate_up_silu_w8a16(x, qg, sg, qu, su, out_dtype=F32)
    assert got16.shape == (rows, n) and got16.dtype == dt
    same = _check(orc, x, qg, sg, qu, su, got16, got32)
    print(f"int8 gate_up [{rows}x{k}] x 2 [{n}x{k}] {dt}: {same:.5f} equal to the oracle")


def test_misaligned_input_takes_the_generic_kernel(pkg, orc, cuda):
    rows, k, n = 9, 256, 64
    x, qg, sg, qu, su = _inputs(rows, k + 1, n, F16, 77, cuda, pkg)
    xv = x[:, 1:]                                  # 2-byte offset: not 16-byte aligned
    qgv, quv = qg[:, 1:], qu[:, 1:]
    got16 = pkg.fused_gate_up_silu_w8a16(xv, qgv, sg, quv, su)
    got32 = pkg.fused_gate_up_silu_w8a16(xv, qgv, sg, quv, su, out_dtype=F32)
    _check(orc, xv.contiguous(), qgv.contiguous(), sg, quv.contiguous(), su, got16, got32)


@pytest.mark.parametrize("rows", [8, 256])
def test_closer_to_exact_than_the_unfused_chain(pkg, orc, cuda, rows):
    k, n = 1536, 2048
    x, qg, sg, qu, su = _inputs(rows, k, n, F16, 5, cuda, pkg)
    fused = pkg.fused_gate_up_silu_w8a16(x, qg, sg, qu, su).double().cpu().numpy()
    chain = pkg.fused_silu_mul(pkg.w8a16_linear(x, qg, sg), pkg.w8a16_linear(x, qu, su)).double().cpu().numpy()
    exact = orc.gate_up_silu_w8a16(storage(x), qg.cpu().numpy(), sg.cpu().numpy(), qu.cpu().numpy(),
                                   su.cpu().numpy(), xdt="f16")["out64"]
    e_fused, e_chain = np.abs(fused - exact).mean(), np.abs(chain - exact).mean()
    print(f"rows {rows}: mean |err| fused {e_fused:.3e}, unfused chain {e_chain:.3e}")
    assert e_fused < e_chain


@pytest.mark.parametrize("rows,k,n", [(8, 1536, 8960), (16, 1536, 8960), (512, 1536, 8960), (24, 896, 4864),
                                      (48, 896, 4864), (4, 896, 4864)])
def test_graph_replays_match_eager(pkg, cuda, rows, k, n):
    x, qg, sg, qu, su = _inputs(rows, k, n, BF16, 9, cuda, pkg)
    xs = x.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pkg.fused_gate_up_silu_w8a16(xs, qg, sg, qu, su)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = pkg.fused_gate_up_silu_w8a16(xs, qg, sg, qu, su)
    for i in range(4):
        xs.copy_(x * (1 + 0.25 * i))
        graph.replay()
        torch.cuda.synchronize()
        want = pkg.fused_gate_up_silu_w8a16(xs, qg, sg, qu, su)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i} differs from eager"


@pytest.mark.parametrize("rows,k,n,dt", [
    (2048, 3584, 4736, BF16),   # 128 x 64 tiles on the sub-step ring
    (1024, 1536, 18944, BF16),  # 256 x 128 tiles on the ring
    (1030, 272, 18900, F16),    # 256 x 128, ragged rows and n, k tail
])
def test_prefill_shape_against_torch_fp64(pkg, cuda, rows, k, n, dt):
    x, qg, sg, qu, su = _inputs(rows, k, n, dt, 21, cuda, pkg)
    got16 = pkg.fused_gate_up_silu_w8a16(x, qg, sg, qu, su).double()
    got32 = pkg.fused_gate_up_silu_w8a16(x, qg, sg, qu, su, out_dtype=F32).double()
    x64 = x.double()
    g = (x64 @ qg.double().T) * sg.double()
    u = (x64 @ qu.double().T) * su.double()
    gabs = (x64.abs() @ qg.double().abs().T) * sg.double().abs()
    uabs = (x64.abs() @ qu.double().abs().T) * su.double().abs()
    exact = torch.nn.functional.silu(g) * u
    bound = torch.from_numpy(act_error_bound(g.cpu().numpy(), u.cpu().numpy(), gabs.cpu().numpy(),
                                             uabs.cpu().numpy(), k)).to(cuda)
    ulp = torch.from_numpy(ulp16(exact.cpu().numpy(), dt)).to(cuda)
    assert float(((got32 - exact).abs() - (2.0 ** -22 * exact.abs() + bound)).max()) <= 1e-30
    assert float(((got16 - exact).abs() - (ulp + bound + 2.0 ** -22 * exact.abs())).max()) <= 0
    assert torch.equal(got16.to(dt), got32.to(dt))


def test_tiled_launch_shapes_agree_bitwise(pkg, cuda):
    """The dual tiled shapes (64 .. 1024 rows of a 7B-wide MLP: 64 x 64, the
    step pipeline's 128 x 64, 128 x 64 and 256 x 128 on the sub-step ring)
    add the k products in the same order: row prefixes give the same bits."""
    rows, k, n = 1024, 1536, 18944
    x, qg, sg, qu, su = _inputs(rows, k, n, F16, 31, cuda, pkg)
    full = pkg.fused_gate_up_silu_w8a16(x, qg, sg, qu, su, out_dtype=F32)
    for r in (64, 256, 257):
        part = pkg.fused_gate_up_silu_w8a16(x[:r], qg, sg, qu, su, out_dtype=F32)
        assert torch.equal(part, full[:r]), f"{r} rows differ from the {rows}-row launch"


def test_quantized_fused_mlp_takes_the_int8_kernel(pkg, cuda, monkeypatch):
    pytest.importorskip("transformers")
    from transformers import Qwen2Config, Qwen2ForCausalLM
    patch_mod = importlib.import_module("llm-inference-optimizer_amd.engine.fused_norm_activation_patch")
    cfg = Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=1024, num_hidden_layers=4,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=128)
    torch.manual_seed(0)
    base = Qwen2ForCausalLM(cfg).to(device=cuda, dtype=F16).eval()
    fused = Qwen2ForCausalLM(cfg).to(device=cuda, dtype=F16).eval()
    fused.load_state_dict(base.state_dict())
    pkg.quantize_model_int8(base)
    counts = pkg.patch_model_with_fused_kernels(fused, fuse_gate_up=True)   # patched first ...
    pkg.quantize_model_int8(fused)                                           # ... then quantised
    assert counts["gate_up"] == 4
    assert all(m.gate_up_kind() == "int8" for m in fused.modules() if isinstance(m, pkg.FusedMLP))
    calls = []
    real = patch_mod.fused_gate_up_silu_w8a16

    def counting(*a, **kw):
        calls.append(a[0].shape)
        return real(*a, **kw)

    monkeypatch.setattr(patch_mod, "fused_gate_up_silu_w8a16", counting)
    ids = torch.randint(0, 512, (2, 40), device=cuda)
    with torch.inference_mode():
        for seq in (8, 40):                       # 16 rows (decode kernel), 80 rows (tiled)
            a = base(ids[:, :seq]).logits.float()
            b = fused(ids[:, :seq]).logits.float()
            err = (a - b).abs().max().item()
            assert err <= 0.05 * a.abs().max().item(), err
    assert len(calls) == 8
