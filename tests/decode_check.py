"""Independent check of a greedy decode, for the graph-captured decoder tests.

The graph-captured decoder (engine/graphed_decode.py) keeps its KV cache in
HF's StaticCache and pins the cache's write position itself every step.  The
check here shares none of that: one prefill of the whole decoded sequence
(the prompt and every generated token but the last) through the model, into
HF's DynamicCache.  That single pass gives

* the key/value the cache must hold at every position -- compared slot by
  slot with the decoder's StaticCache after its last step.  A token written
  one slot off, a stale slot or a wrong position id shows up as an O(1)
  relative error at exactly those slots, far above rounding;
* the logits that predict every generated token -- compared with the logits
  the decoder used (``return_logits=True``), and each generated token must be
  the greedy pick of these independent logits except where their top two are
  within the observed rounding noise (a near-tie).

Random-init models attend almost uniformly, which blunts a logit-level check;
the cache comparison does not depend on it, and ``sharpen_attention`` scales
the query / key projections so the logits are position-sensitive too.
"""
from __future__ import annotations

import torch


def sharpen_attention(model, factor: float) -> None:
    """Scale every layer's query and key projections (weights and biases) by
    `factor`: attention scores grow by factor**2."""
    with torch.no_grad():
        for layer in model.model.layers:
            for proj in (layer.self_attn.q_proj, layer.self_attn.k_proj):
                proj.weight.mul_(factor)
                if proj.bias is not None:
                    proj.bias.mul_(factor)


def reference_pass(model, prompt: torch.Tensor, new_tokens: torch.Tensor):
    """One prefill of ``prompt`` followed by ``new_tokens[:, :-1]`` into a
    DynamicCache.  Returns (fp32 logits [B, NEW, vocab] that predict each of
    the NEW tokens, the filled DynamicCache)."""
    from transformers import DynamicCache

    seq = torch.cat([prompt, new_tokens[:, :-1]], dim=1)
    with torch.inference_mode():
        cache = DynamicCache(config=model.config)
        out = model(input_ids=seq, past_key_values=cache, use_cache=True)
    return out.logits[:, prompt.shape[1] - 1:].float(), cache


def cache_slot_error(static_cache, dynamic_cache) -> tuple[float, list[int]]:
    """Largest relative difference between the two caches' keys and values,
    over layers, at every position the dynamic cache holds (relative to the
    largest magnitude of that layer's tensor), and the positions where it
    exceeds 5%."""
    worst = 0.0
    bad = set()
    for ls, ld in zip(static_cache.layers, dynamic_cache.layers):
        n = ld.keys.shape[2]
        for s, d in ((ls.keys[:, :, :n], ld.keys), (ls.values[:, :, :n], ld.values)):
            per_slot = (s.float() - d.float()).abs().amax(dim=(0, 1, 3)) / d.float().abs().max()
            worst = max(worst, per_slot.max().item())
            bad.update((per_slot > 0.05).nonzero().flatten().tolist())
    return worst, sorted(bad)


def compare_logits(new_tokens: torch.Tensor, logits: torch.Tensor, ref_logits: torch.Tensor) -> dict:
    """Agreement of a decode (its generated tokens and the logits behind
    them) with independently computed logits for the same tokens."""
    noise = (logits - ref_logits).abs().max().item()
    ref_pick = ref_logits.argmax(-1)
    differ = ref_pick != new_tokens
    top2 = ref_logits.topk(2, dim=-1).values
    gap = top2[..., 0] - top2[..., 1]
    return {
        "noise": noise,
        "logit_scale": ref_logits.abs().max().item(),
        "mismatch_frac": differ.float().mean().item(),
        "max_gap_at_mismatch": gap[differ].max().item() if differ.any() else 0.0,
        "median_gap": gap.median().item(),
    }


def check_decode(model, dec, prompt, out, logits, logit_tol: float, cache_tol: float, what: str) -> dict:
    """Checks a finished ``dec.generate(prompt, NEW, return_logits=True)``
    (tokens ``out``, logits ``logits``) against the reference pass; the
    decoder's StaticCache must still hold this generation's keys/values."""
    n = prompt.shape[1]
    new = out[:, n:]
    ref_logits, ref_cache = reference_pass(model, prompt, new)
    r = compare_logits(new, logits, ref_logits)
    r["cache_err"], r["bad_slots"] = cache_slot_error(dec.cache, ref_cache)
    print(f"{what}: cache max rel error {r['cache_err']:.3g} (bad slots {r['bad_slots'][:8]}); "
          f"max |dlogit| {r['noise']:.4g} (logit scale {r['logit_scale']:.3g}); greedy token != independent "
          f"argmax for {r['mismatch_frac']:.2%} (largest independent top-2 gap there {r['max_gap_at_mismatch']:.4g}, "
          f"median gap {r['median_gap']:.4g})")
    assert r["cache_err"] <= cache_tol, f"{what}: cache slots {r['bad_slots']} differ (max rel {r['cache_err']:.3g})"
    assert r["noise"] <= logit_tol, f"{what}: logits differ by {r['noise']:.4g} > {logit_tol}"
    assert r["max_gap_at_mismatch"] <= 2 * r["noise"] + 1e-6, f"{what}: a token differs away from a near-tie"
    return r
