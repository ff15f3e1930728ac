"""Graph-captured decode caller (the reference's Stage 6 GraphedDecodeEngine,
src/engine/graphed_decode_engine.py, rebuilt on HF's StaticCache), checked as
the reference checks its engine (tests/test_graphed_decode.py:49-102):

* the graphed decode of the 28-layer Qwen2 -- patched with the fused RMSNorm
  / SiLU-and-mul kernels and unpatched, each on a freshly built model -- must
  agree with an independent computation that shares none of the decoder's
  cache logic: one prefill of the decoded sequence into HF's DynamicCache
  (tests/decode_check.py).  Every key/value slot of the decoder's StaticCache
  must match it to fp16 rounding, the logits behind every generated token
  must match to fp16 noise, and every token must be the independent greedy
  pick except at a near-tie.  A cache slot written at the wrong position
  shows up as an O(1) relative error at that slot (the CPU test
  test_graphed_decode_cpu.py plants exactly that mistake and checks the
  tolerances below catch it);
* a second, different prompt, of another length, decoded through the
  already-captured graph (no recapture) must pass the same check;
* the same static-cache step run eagerly gives the same tokens and logits
  bit for bit (graph capture changes nothing).

Random-init weights attend almost uniformly, which would blunt the position
check, so the query / key projections are scaled up (tests/decode_check.py,
sharpen_attention).
"""
import pytest
import torch

from decode_check import check_decode, sharpen_attention

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")

B, S, NEW = 4, 64, 48
S2 = 55  # the second prompt's length
# fp16 rounding between the graphed decode and one prefill of the same
# tokens: differently shaped attention and GEMM computations (one token
# against a masked max_cache_len cache vs the whole sequence at once) through
# 28 layers.  Logits: max |difference| (0.11 measured against an
# incremental DynamicCache decode, on a logit scale of 4.2).  Cache: max
# difference of a slot relative to the layer's largest key / value (a slot
# written one position off: ~1; measured here: at most 0.032).
LOGIT_TOL = 0.25
CACHE_TOL = 0.1


def _model(cuda, seed=3, layers=28, vocab=151936):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    cfg = Qwen2Config(vocab_size=vocab, hidden_size=1536, intermediate_size=8960, num_hidden_layers=layers,
                      num_attention_heads=12, num_key_value_heads=2, max_position_embeddings=4096,
                      rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True, attn_implementation="sdpa")
    torch.manual_seed(seed)
    with torch.device(cuda):
        m = Qwen2ForCausalLM(cfg)
    m = m.half().eval()
    sharpen_attention(m, 3.0)
    return m


def _prompt(cuda, vocab, seed, length):
    g = torch.Generator()
    g.manual_seed(seed)
    return torch.randint(0, vocab, (B, length), generator=g).to(cuda)


def _check_against_dynamic_cache(model, dec, ids, out, logits, what):
    n = ids.shape[1]
    assert torch.equal(out[:, :n], ids)
    assert torch.equal(logits.argmax(-1), out[:, n:])
    return check_decode(model, dec, ids, out, logits, LOGIT_TOL, CACHE_TOL, what)


@pytest.mark.parametrize("patched", [False, True])
def test_graph_decode_matches_independent_dynamic_cache_decode(pkg, cuda, patched):
    model = _model(cuda)  # fresh for each case: patching replaces modules in place
    if patched:
        assert pkg.patch_model_with_fused_kernels(model) == {"rmsnorm": 57, "mlp": 28}
        assert isinstance(model.model.layers[0].mlp, pkg.FusedMLP)
    vocab = model.config.vocab_size
    dec = pkg.GraphedGreedyDecoder(model, B, S + NEW + 8)

    ids = _prompt(cuda, vocab, 11, S)
    out, logits = dec.generate(ids, NEW, return_logits=True)
    graph = dec._graph
    assert graph is not None
    _check_against_dynamic_cache(model, dec, ids, out, logits, f"patched={patched} prompt A")

    # the identical static-cache step, eager: graph capture changes nothing
    eager_out, eager_logits = pkg.GraphedGreedyDecoder(model, B, S + NEW + 8, use_graph=False).generate(
        ids, NEW, return_logits=True)
    assert torch.equal(out, eager_out) and torch.equal(logits, eager_logits)

    # a different prompt of another length through the already-captured graph
    ids2 = _prompt(cuda, vocab, 12, S2)
    out2, logits2 = dec.generate(ids2, NEW, return_logits=True)
    assert dec._graph is graph, "the second generation must replay the captured graph, not recapture"
    _check_against_dynamic_cache(model, dec, ids2, out2, logits2, f"patched={patched} prompt B (reused graph)")
    assert not torch.equal(out2[:, S2:], out[:, S:S + NEW])

    # and the first prompt again through the same graph reproduces its decode
    again, again_logits = dec.generate(ids, NEW, return_logits=True)
    assert torch.equal(again, out) and torch.equal(again_logits, logits)
    del dec, model
    torch.cuda.empty_cache()


def test_graph_decode_with_every_fused_kernel_matches_independent_decode(pkg, cuda):
    """A model patched with every opt-in kernel (residual add + RMSNorm,
    gate/up + SiLU-and-mul, the HIP down projection) decodes, with its step
    replayed as one HIP graph, what the independent DynamicCache decode
    confirms, and the same tokens as the eager static-cache step."""
    m = _model(cuda, seed=5, layers=4, vocab=4096)
    counts = pkg.patch_model_with_fused_kernels(m, fuse_residual=True, fuse_gate_up=True, hip_down=True)
    assert counts == {"rmsnorm": 9, "mlp": 4, "gate_up": 4, "down": 4, "add_rmsnorm": 4}
    ids = _prompt(cuda, 4096, 11, S)
    dec = pkg.GraphedGreedyDecoder(m, B, S + NEW + 8)
    out, logits = dec.generate(ids, NEW, return_logits=True)
    assert dec._graph is not None
    _check_against_dynamic_cache(m, dec, ids, out, logits, "every fused kernel")
    eager = pkg.GraphedGreedyDecoder(m, B, S + NEW + 8, use_graph=False).generate(ids, NEW)
    assert torch.equal(out, eager)
    ids2 = _prompt(cuda, 4096, 12, S2)
    out2, logits2 = dec.generate(ids2, NEW, return_logits=True)
    _check_against_dynamic_cache(m, dec, ids2, out2, logits2, "every fused kernel, prompt B (reused graph)")
