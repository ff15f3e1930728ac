"""CPU checks of the graph-captured decoder's step logic and of the
independent checker its GPU test relies on (tests/decode_check.py).

A small random-init Qwen2 in fp32 on the CPU runs GraphedGreedyDecoder's
static-cache step eagerly (``use_graph=False``; the graph only replays this
step).  Its cache and logits must agree with one DynamicCache prefill of the
decoded sequence to fp32 rounding, for two different prompts of different
lengths through one decoder object (its static buffers reused).  And a
decoder that writes each token's key/value one cache slot early -- the kind
of mistake the step's position pinning could make -- must be flagged by the
same check, at exactly the decode slots.
"""
import pytest
import torch

from decode_check import check_decode, sharpen_attention

transformers = pytest.importorskip("transformers")

B, NEW = 2, 12


@pytest.fixture(scope="module")
def tiny():
    from transformers import Qwen2Config, Qwen2ForCausalLM
    cfg = Qwen2Config(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=4,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512,
                      rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True, attn_implementation="sdpa")
    torch.manual_seed(7)
    m = Qwen2ForCausalLM(cfg).float().eval()
    sharpen_attention(m, 8.0)
    return m


def _prompt(seed, S, vocab):
    g = torch.Generator()
    g.manual_seed(seed)
    return torch.randint(0, vocab, (B, S), generator=g)


def test_static_cache_step_matches_dynamic_cache(pkg, tiny):
    dec = pkg.GraphedGreedyDecoder(tiny, B, 64, use_graph=False)
    for seed, S in ((1, 24), (2, 17)):  # the second prompt reuses the decoder's static buffers
        ids = _prompt(seed, S, tiny.config.vocab_size)
        out, logits = dec.generate(ids, NEW, return_logits=True)
        assert torch.equal(out[:, :S], ids) and out.shape == (B, S + NEW)
        assert torch.equal(logits.argmax(-1), out[:, S:])
        r = check_decode(tiny, dec, ids, out, logits, logit_tol=1e-4, cache_tol=1e-5, what=f"cpu prompt {seed}")
        assert r["mismatch_frac"] == 0.0


class OneSlotEarly:
    """Mixin: pins the cache's write counter one slot before the token's
    position, so each token's key/value overwrite the previous token's."""

    def _step(self):
        counters = [layer.cumulative_length for layer in self.cache.layers]
        early = self._pos0 - 1
        torch._foreach_copy_(counters, [early] * len(counters))
        out = self.model(input_ids=self._tok, past_key_values=self.cache, cache_position=self._pos,
                         position_ids=self._pos_ids, use_cache=True)
        logits = out.logits[:, -1]
        return logits, logits.argmax(-1, keepdim=True)


def test_checker_flags_a_misplaced_cache_slot(pkg, tiny):
    broken = type("Broken", (OneSlotEarly, pkg.GraphedGreedyDecoder), {})
    S = 24
    ids = _prompt(1, S, tiny.config.vocab_size)
    dec = broken(tiny, B, 64, use_graph=False)
    out, logits = dec.generate(ids, NEW, return_logits=True)
    with pytest.raises(AssertionError, match="cache slots"):
        # the GPU test's tolerances: the mistake is caught even there
        check_decode(tiny, dec, ids, out, logits, logit_tol=0.25, cache_tol=0.1, what="planted mistake")
    from decode_check import cache_slot_error, reference_pass
    _, ref_cache = reference_pass(tiny, ids, out[:, S:])
    err, bad = cache_slot_error(dec.cache, ref_cache)
    print(f"one slot early: cache max rel error {err:.3g} at slots {bad}")
    assert err > 0.3 and bad == list(range(S - 1, S + NEW - 1))
