"""GPU checks of the fused residual add + RMSNorm (beyond the reference; the
"fused RMSNorm + residual" its design plans, docs/architecture-cuda.md:94):

* parity with the oracle's restatement (h bit-exact, y within 1 ulp) over
  the BASELINE widths, decode rows, odd widths and dtype mixes;
* bit-identity with the unfused composition `h = residual + x` (torch's
  add) followed by `fused_rmsnorm(h)` -- the property that makes the fused
  decoder layer a drop-in;
* in-place use through the C ABI and the fp32-value tolerance;
* a 28-layer Qwen2 patched with fuse_residual=True produces logits bit-
  identical to the same model patched without it.
"""
import importlib

import numpy as np
import pytest
import torch

from parity_utils import DT_NAME, randn, storage, ulp_report

pytestmark = pytest.mark.gpu

F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32


def _lib():
    return importlib.import_module("llm-inference-optimizer_amd._lib")


@pytest.mark.parametrize("rows,n,dt,wdt", [
    (2048, 1536, F16, F16), (16384, 3584, BF16, BF16),
    (1, 1536, F16, F16), (8, 1536, F16, F16), (32, 1536, F16, F16),
    (7, 100, F16, F16), (5, 8200, BF16, BF16), (9, 896, F16, F32), (6, 2048, F32, F32), (3, 40000, BF16, BF16),
    # from 1024 rows up a wave holds two rows: an odd count leaves a lone row
    (1025, 1536, F16, F16), (2049, 2048, F16, F32), (1031, 896, BF16, BF16),
])
def test_add_rmsnorm_matches_oracle(pkg, orc, cuda, rows, n, dt, wdt):
    x = randn((rows, n), 50, dt)
    r = randn((rows, n), 51, dt, std=4.0)
    w = randn((n,), 52, wdt, mean=1.0, std=0.1)
    y, h = pkg.fused_add_rmsnorm(x.to(cuda), r.to(cuda), w.to(cuda), 1e-6)
    y, h = y.cpu(), h.cpu()
    yo, ho = orc.add_rmsnorm(storage(x), storage(r), storage(w), 1e-6, xdt=DT_NAME[dt], wdt=DT_NAME[wdt],
                             ydt=DT_NAME[dt])
    assert np.array_equal(storage(h), ho), "residual out differs from round(x + r)"
    if dt == F32:
        np.testing.assert_allclose(y.numpy(), yo, rtol=2e-6, atol=1e-30)
    else:
        mx, frac = ulp_report(storage(y), yo, orc)
        print(f"add_rmsnorm [{rows},{n}] {dt}: max ulp {mx}, mismatched {frac:.2e}")
        assert mx <= 1 and frac < 0.01


@pytest.mark.parametrize("rows,n,dt", [(2048, 1536, F16), (16384, 3584, BF16), (8, 1536, F16),
                                       (7, 100, F16), (5, 8200, BF16), (1027, 1536, F16)])
def test_add_rmsnorm_equals_add_then_norm(pkg, cuda, rows, n, dt):
    x = randn((rows, n), 60, dt).to(cuda)
    r = randn((rows, n), 61, dt, std=4.0).to(cuda)
    w = randn((n,), 62, dt, mean=1.0, std=0.1).to(cuda)
    y1, h1 = pkg.fused_add_rmsnorm(x, r, w, 1e-6)
    h2 = r + x
    y2 = pkg.fused_rmsnorm(h2, w, 1e-6)
    assert torch.equal(h1, h2)
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("rows", [64, 1025])
def test_add_rmsnorm_in_place_through_abi(pkg, cuda, rows):
    """residual_out = residual and y = x (the in-place form a decoder loop
    uses): same bits as the out-of-place call, also where each wave holds two
    rows (1025 rows: the last wave holds one)."""
    L = _lib()
    n = 1536
    x = randn((rows, n), 70, F16).to(cuda)
    r = randn((rows, n), 71, F16).to(cuda)
    w = randn((n,), 72, F16, mean=1.0, std=0.1).to(cuda)
    y_ref, h_ref = pkg.fused_add_rmsnorm(x, r, w, 1e-6)
    L.add_rmsnorm_fwd(x.data_ptr(), r.data_ptr(), w.data_ptr(), x.data_ptr(), r.data_ptr(), rows, n, n, n, n, n,
                      1e-6, L.F16, L.F16, L.F16, L.stream_handle(cuda))
    torch.cuda.synchronize()
    assert torch.equal(x, y_ref) and torch.equal(r, h_ref)


def test_add_rmsnorm_strided_and_misaligned(pkg, orc, cuda):
    base_x = randn((32, 2048), 80, F16)
    base_r = randn((32 * 1536 + 1,), 81, F16)
    w = randn((1536,), 82, F16, mean=1.0, std=0.1)
    xv = base_x.to(cuda)[:, 128:128 + 1536]          # row-strided view
    rv = base_r.to(cuda)[1:].view(32, 1536)          # misaligned -> generic kernel
    y, h = pkg.fused_add_rmsnorm(xv, rv, w.to(cuda))
    yo, ho = orc.add_rmsnorm(storage(base_x[:, 128:128 + 1536]), storage(base_r[1:].view(32, 1536)), storage(w),
                             1e-6, xdt="f16", wdt="f16")
    assert np.array_equal(storage(h.cpu()), ho)
    mx, frac = ulp_report(storage(y.cpu()), yo, orc)
    assert mx <= 1 and frac < 0.01


def test_add_rmsnorm_fp32_value_within_tolerance(orc, cuda):
    L = _lib()
    rows, n = 64, 3584
    x = randn((rows, n), 90, BF16).to(cuda)
    r = randn((rows, n), 91, BF16).to(cuda)
    w = randn((n,), 92, BF16, mean=1.0, std=0.1).to(cuda)
    y = torch.empty((rows, n), dtype=F32, device=cuda)
    h = torch.empty_like(x)
    L.add_rmsnorm_fwd(x.data_ptr(), r.data_ptr(), w.data_ptr(), y.data_ptr(), h.data_ptr(), rows, n, n, n, n, n,
                      1e-6, L.BF16, L.BF16, L.F32, L.stream_handle(cuda))
    ref = orc.rmsnorm_f64(storage(h.cpu()), storage(w.cpu()), 1e-6, xdt="bf16", wdt="bf16")
    err = np.abs(y.cpu().numpy().astype(np.float64) - ref)
    assert (err <= 1e-3 + 1e-3 * np.abs(ref)).all()
    assert (err <= 1e-30 + 1e-5 * np.abs(ref)).all()


def test_fused_decoder_layers_bit_identical(pkg, cuda):
    transformers = pytest.importorskip("transformers")
    from transformers import Qwen2Config, Qwen2ForCausalLM
    cfg = Qwen2Config(vocab_size=151936, hidden_size=1536, intermediate_size=8960, num_hidden_layers=28,
                      num_attention_heads=12, num_key_value_heads=2, max_position_embeddings=4096,
                      rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True, attn_implementation="sdpa")
    torch.manual_seed(1)
    with torch.device(cuda):
        model = Qwen2ForCausalLM(cfg)
    model = model.half().eval()
    g = torch.Generator()
    g.manual_seed(9)
    ids = torch.randint(0, cfg.vocab_size, (2, 128), generator=g).to(cuda)
    assert pkg.patch_model_with_fused_kernels(model) == {"rmsnorm": 57, "mlp": 28}
    with torch.inference_mode():
        want = model(input_ids=ids).logits
    counts = pkg.patch_model_with_fused_kernels(model, fuse_residual=True)
    assert counts["add_rmsnorm"] == 28
    assert isinstance(model.model.layers[5], pkg.FusedDecoderLayer)
    with torch.inference_mode():
        got = model(input_ids=ids).logits
        # and with a KV cache: prefill then one decode step
        out = model(input_ids=ids, use_cache=True)
        step = model(input_ids=out.logits[:, -1:].argmax(-1), past_key_values=out.past_key_values, use_cache=True)
    assert torch.equal(got, want)
    assert torch.isfinite(step.logits).all()
