"""End-to-end checks of the weight-only int8 stage, after the reference's
tests/test_e2e_quantization.py, on a random-init Qwen2 of the BASELINE
config-5 architecture (28 layers, hidden 1536, intermediate 8960, 12 / 2
heads, vocab 151936, fp16; the reference loads Qwen2.5-1.5B-Instruct from the
Hub, which is not reachable here):

1. the quantiser replaces 7 linears per layer (196), the first q_proj is a
   QuantizedLinearInt8, and the layer bytes drop below 60%;
2. quantised logits stay close to fp16 (mean cosine > 0.99, top-1 agreement
   >= 80%, the reference's bars) -- on a prompt of uniform token ids;
3. composition: the quantised model, also patched with the fused RMSNorm /
   SiLU-and-mul kernels, decodes the same tokens with the graph-captured
   decoder as with the eager static-cache step (same weights on both sides,
   so exact agreement is the bar, as in the reference's PagedEngine check).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")


def _model(cuda, layers=28, seed=0):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    cfg = Qwen2Config(vocab_size=151936, hidden_size=1536, intermediate_size=8960, num_hidden_layers=layers,
                      num_attention_heads=12, num_key_value_heads=2, max_position_embeddings=4096,
                      rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True, initializer_range=0.02,
                      attn_implementation="sdpa")
    torch.manual_seed(seed)
    with torch.device(cuda):
        m = Qwen2ForCausalLM(cfg)
    return m.half().eval()


def _ids(cuda, vocab, B, S, seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return torch.randint(0, vocab, (B, S), generator=g).to(cuda)


def test_quantizer_actually_replaces_layers(pkg, cuda):
    model = _model(cuda)
    stats = pkg.quantize_model_int8(model)
    num_layers = model.config.num_hidden_layers
    assert stats["layers_quantized"] == num_layers * 7, stats
    assert isinstance(model.model.layers[0].self_attn.q_proj, pkg.QuantizedLinearInt8)
    assert stats["bytes_after"] < 0.6 * stats["bytes_before"]
    assert not any(isinstance(m, torch.nn.Linear) for m in model.model.layers.modules())
    assert isinstance(model.lm_head, torch.nn.Linear)          # lm_head / embeddings untouched (tied)
    print(f"quantize stats: {stats}")


def test_quantized_logits_close_to_fp16(pkg, cuda):
    model = _model(cuda, seed=1)
    ids = _ids(cuda, model.config.vocab_size, 1, 96, seed=2)
    with torch.inference_mode():
        fp16_logits = model(input_ids=ids).logits.float()
    pkg.quantize_model_int8(model)
    with torch.inference_mode():
        int8_logits = model(input_ids=ids).logits.float()
    assert not torch.isnan(int8_logits).any(), "quantized model produced NaN"
    cosine = torch.nn.functional.cosine_similarity(fp16_logits, int8_logits, dim=-1)
    agreement = (fp16_logits.argmax(-1) == int8_logits.argmax(-1)).float().mean().item()
    print(f"int8 vs fp16: mean cosine {cosine.mean().item():.5f}, top-1 agreement {agreement:.1%}")
    assert cosine.mean().item() > 0.99
    assert agreement >= 0.8


def test_quantized_and_fused_model_graph_decode_matches_eager(pkg, cuda):
    model = _model(cuda, seed=3)
    stats = pkg.quantize_model_int8(model)
    counts = pkg.patch_model_with_fused_kernels(model)
    assert stats["layers_quantized"] == 196 and counts == {"rmsnorm": 57, "mlp": 28}
    assert isinstance(model.model.layers[0].mlp.gate_proj, pkg.QuantizedLinearInt8)
    B, S, NEW = 4, 48, 32
    ids = _ids(cuda, model.config.vocab_size, B, S, seed=4)
    eager = pkg.GraphedGreedyDecoder(model, B, S + NEW + 8, use_graph=False).generate(ids, NEW)
    dec = pkg.GraphedGreedyDecoder(model, B, S + NEW + 8)
    graphed = dec.generate(ids, NEW)
    assert dec._graph is not None
    assert torch.equal(graphed, eager)
