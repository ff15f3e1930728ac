"""Module-replacement plugin behaviour (host-only; no kernel runs): the same
matching, counting, toggles and parameter sharing as the reference's
src/engine/fused_norm_activation_patch.py:29-99, on random-init
transformers models built locally."""
import pytest
import torch

transformers = pytest.importorskip("transformers")


def _qwen2(layers=28, hidden=64, inter=128):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    cfg = Qwen2Config(vocab_size=128, hidden_size=hidden, intermediate_size=inter, num_hidden_layers=layers,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
    return Qwen2ForCausalLM(cfg)


def test_patch_counts_on_28_layer_qwen2(pkg):
    model = _qwen2()
    counts = pkg.patch_model_with_fused_kernels(model)
    # 2 norms per layer + final norm; 1 MLP per layer (benchmarks/results/stage3_e2e.json:2-3)
    assert counts == {"rmsnorm": 57, "mlp": 28}
    layer = model.model.layers[0]
    assert isinstance(layer.input_layernorm, pkg.FusedRMSNorm)
    assert isinstance(layer.post_attention_layernorm, pkg.FusedRMSNorm)
    assert isinstance(layer.mlp, pkg.FusedMLP)
    assert isinstance(model.model.norm, pkg.FusedRMSNorm)
    # patching twice finds nothing new: the replacements are not matched again
    assert pkg.patch_model_with_fused_kernels(model) == {"rmsnorm": 0, "mlp": 0}


def test_replacements_share_parameters(pkg):
    model = _qwen2(layers=2)
    norm = model.model.layers[1].post_attention_layernorm
    mlp = model.model.layers[1].mlp
    w, eps = norm.weight, norm.variance_epsilon
    gp, up, dp = mlp.gate_proj, mlp.up_proj, mlp.down_proj
    n_params = sum(p.numel() for p in model.parameters())
    pkg.patch_model_with_fused_kernels(model)
    fn = model.model.layers[1].post_attention_layernorm
    fm = model.model.layers[1].mlp
    assert fn.weight is w and fn.variance_epsilon == eps
    assert fm.gate_proj is gp and fm.up_proj is up and fm.down_proj is dp
    assert not hasattr(fm, "act_fn")
    assert sum(p.numel() for p in model.parameters()) == n_params
    assert dict(model.named_parameters()).keys() == dict(_qwen2(layers=2).named_parameters()).keys()


@pytest.mark.parametrize("norm,mlp,want", [(True, False, {"rmsnorm": 9, "mlp": 0}),
                                           (False, True, {"rmsnorm": 0, "mlp": 4}),
                                           (False, False, {"rmsnorm": 0, "mlp": 0})])
def test_patch_toggles(pkg, norm, mlp, want):
    model = _qwen2(layers=4)
    assert pkg.patch_model_with_fused_kernels(model, patch_norm=norm, patch_mlp=mlp) == want


def test_llama_names_match(pkg):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=64, hidden_size=32, intermediate_size=64, num_hidden_layers=3,
                      num_attention_heads=4, num_key_value_heads=2)
    counts = pkg.patch_model_with_fused_kernels(LlamaForCausalLM(cfg))
    assert counts == {"rmsnorm": 7, "mlp": 3}


def test_unrecognised_architecture_patches_nothing(pkg):
    model = torch.nn.Sequential(torch.nn.Linear(8, 8), torch.nn.LayerNorm(8), torch.nn.GELU())
    assert pkg.patch_model_with_fused_kernels(model) == {"rmsnorm": 0, "mlp": 0}


def test_class_name_sets_match_reference(pkg):
    assert pkg.RMSNORM_CLASS_NAMES == {"Qwen2RMSNorm", "LlamaRMSNorm", "MistralRMSNorm", "RMSNorm"}
    assert pkg.MLP_CLASS_NAMES == {"Qwen2MLP", "LlamaMLP", "MistralMLP"}


def test_matching_requires_attributes(pkg):
    class RMSNorm(torch.nn.Module):  # right name, missing variance_epsilon
        def __init__(self):
            super().__init__()
            self.weight = torch.nn.Parameter(torch.ones(4))

    class Qwen2MLP(torch.nn.Module):  # right name, missing down_proj
        def __init__(self):
            super().__init__()
            self.gate_proj = torch.nn.Linear(4, 8)
            self.up_proj = torch.nn.Linear(4, 8)

    root = torch.nn.Module()
    root.norm = RMSNorm()
    root.mlp = Qwen2MLP()
    assert pkg.patch_model_with_fused_kernels(root) == {"rmsnorm": 0, "mlp": 0}


def test_fuse_residual_replaces_decoder_layers(pkg):
    model = _qwen2(layers=28)
    attn0 = model.model.layers[0].self_attn
    counts = pkg.patch_model_with_fused_kernels(model, fuse_residual=True)
    assert counts == {"rmsnorm": 57, "mlp": 28, "add_rmsnorm": 28}
    layer = model.model.layers[0]
    assert isinstance(layer, pkg.FusedDecoderLayer)
    assert layer.self_attn is attn0
    assert isinstance(layer.input_layernorm, pkg.FusedRMSNorm)
    assert isinstance(layer.post_attention_layernorm, pkg.FusedRMSNorm)
    assert isinstance(layer.mlp, pkg.FusedMLP)
    assert len(model.model.layers) == 28
    # default call keeps the reference's return value exactly
    assert pkg.patch_model_with_fused_kernels(_qwen2(layers=2)) == {"rmsnorm": 5, "mlp": 2}
    assert pkg.DECODER_LAYER_CLASS_NAMES == {"Qwen2DecoderLayer", "LlamaDecoderLayer", "MistralDecoderLayer"}


def test_fuse_gate_up_is_opt_in_and_counted(pkg):
    model = _qwen2(layers=4)
    assert pkg.patch_model_with_fused_kernels(model, fuse_gate_up=True) == {"rmsnorm": 9, "mlp": 4, "gate_up": 4}
    assert all(layer.mlp.fuse_gate_up for layer in model.model.layers)
    plain = _qwen2(layers=2)
    assert pkg.patch_model_with_fused_kernels(plain) == {"rmsnorm": 5, "mlp": 2}
    assert not any(layer.mlp.fuse_gate_up for layer in plain.model.layers)


def test_fuse_gate_up_skips_projections_the_kernel_cannot_read(pkg):
    # k (the hidden size) not a multiple of 8
    odd = _qwen2(layers=2, hidden=60)
    assert pkg.patch_model_with_fused_kernels(odd, fuse_gate_up=True)["gate_up"] == 0
    # projections with a bias, or not plain nn.Linear layers
    model = _qwen2(layers=2)
    mlp0, mlp1 = model.model.layers[0].mlp, model.model.layers[1].mlp
    mlp0.gate_proj = torch.nn.Linear(64, 128, bias=True)

    class QuantLinear(torch.nn.Linear):
        pass

    mlp1.up_proj = QuantLinear(64, 128, bias=False)
    counts = pkg.patch_model_with_fused_kernels(model, fuse_gate_up=True)
    assert counts["mlp"] == 2 and counts["gate_up"] == 0


def test_hip_down_is_opt_in_and_counted(pkg):
    model = _qwen2(layers=4)
    counts = pkg.patch_model_with_fused_kernels(model, hip_down=True)
    assert counts == {"rmsnorm": 9, "mlp": 4, "down": 4}
    assert all(layer.mlp.hip_down for layer in model.model.layers)
    both = _qwen2(layers=2)
    assert pkg.patch_model_with_fused_kernels(both, fuse_gate_up=True, hip_down=True) == {
        "rmsnorm": 5, "mlp": 2, "gate_up": 2, "down": 2}
    plain = _qwen2(layers=2)
    assert pkg.patch_model_with_fused_kernels(plain) == {"rmsnorm": 5, "mlp": 2}
    assert not any(layer.mlp.hip_down for layer in plain.model.layers)


def test_hip_down_skips_down_projections_the_kernel_cannot_run(pkg):
    model = _qwen2(layers=2)

    class QuantLinear(torch.nn.Linear):
        pass

    model.model.layers[0].mlp.down_proj = QuantLinear(128, 64, bias=False)
    counts = pkg.patch_model_with_fused_kernels(model, hip_down=True)
    assert counts["mlp"] == 2 and counts["down"] == 1
    assert not model.model.layers[0].mlp.hip_down and model.model.layers[1].mlp.hip_down


def test_hip_down_leaves_fp32_and_large_inputs_to_the_module(pkg):
    """fp32 activations and inputs above LINEAR16_MAX_ROWS rows call the
    down_proj module itself (so they run on the CPU here, no kernel)."""
    model = _qwen2(layers=1)
    pkg.patch_model_with_fused_kernels(model, hip_down=True)
    mlp = model.model.layers[0].mlp
    act = torch.randn(3, 128)
    assert torch.equal(mlp.down(act), mlp.down_proj(act))
    big = torch.randn(pkg.LINEAR16_MAX_ROWS + 1, 128).half()
    mlp.down_proj.half()
    assert torch.equal(mlp.down(big), mlp.down_proj(big))


def test_quantized_linear_module_host_side(pkg):
    """QuantizedLinearInt8's host-side surface (the reference's interface,
    src/quantization/int8.py:32-63): buffers, sizes, the dense weight the
    codes stand for, and shape checks."""
    codes = torch.tensor([[1, -2, 127], [0, -127, 5]], dtype=torch.int8)
    scale = torch.tensor([0.5, 0.25], dtype=torch.float32)
    bias = torch.tensor([1.0, -1.0], dtype=torch.float16)
    q = pkg.QuantizedLinearInt8(codes, scale, bias)
    assert (q.in_features, q.out_features) == (3, 2)
    assert dict(q.named_buffers()).keys() == {"weight_q", "scale", "bias"} and not list(q.parameters())
    want = torch.tensor([[0.5, -1.0, 63.5], [0.0, -31.75, 1.25]])
    assert torch.equal(q.dequantized_weight(), want)
    assert q.dequantized_weight(torch.float16).dtype == torch.float16
    assert q.num_bytes() == 6 + 8 + 4
    assert pkg.QuantizedLinearInt8(codes, scale, None).num_bytes() == 14
    assert "bias=True" in repr(q)
    with pytest.raises(ValueError):
        pkg.QuantizedLinearInt8(codes.float(), scale, None)
    with pytest.raises(ValueError):
        pkg.QuantizedLinearInt8(codes, scale[:1], None)


def test_quantize_model_without_linears_reports_zero(pkg):
    """A model whose decoder layers hold no nn.Linear is left untouched and
    reports zero replacements (no GPU needed: nothing is quantised)."""
    model = torch.nn.Module()
    model.model = torch.nn.Module()
    model.model.layers = torch.nn.ModuleList([torch.nn.LayerNorm(8) for _ in range(3)])
    assert pkg.quantize_model_int8(model) == {"layers_quantized": 0, "bytes_before": 0, "bytes_after": 0}
