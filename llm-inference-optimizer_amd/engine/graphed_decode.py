"""Greedy decoding whose per-token step replays one captured HIP graph.

The caller the reference's Stage 6 engine provides
(src/engine/graphed_decode_engine.py:47-186, GraphedDecodeEngine), rebuilt on
HF's own ``StaticCache`` instead of the reference's paged KV cache (paged
attention is not on this path): every buffer the decode step touches is
allocated once, the step reads only static tensors (the current tokens and
the cache position), and after the first step the whole forward pass -- 28
layers of attention, the fused RMSNorm / SiLU-and-mul kernels, GEMMs, LM head
and argmax -- is one graph replay.  As in the reference (:129-147), the graph
is replayed right after capture, so the first captured step also returns a
computed result rather than whatever the capture pass left behind.

It works with the patched and the unpatched model alike; the fused kernels
enqueue no allocation, sync or memset, so they capture cleanly.
"""
from __future__ import annotations

import torch

__all__ = ["GraphedGreedyDecoder"]


class GraphedGreedyDecoder:
    """Greedy generation for an HF causal LM with a graph-captured decode step.

    ``batch_size`` and ``max_cache_len`` fix the static buffers (one graph per
    decoder).  ``generate(input_ids, max_new_tokens)`` returns the prompt
    followed by the generated tokens, like ``generate_graphed`` in the
    reference (:177-186); with ``return_logits=True`` it also returns the
    last-position logits behind each generated token, [batch, new, vocab]
    (the prefill's, then each step's).  ``use_graph=False`` runs the
    identical static-cache step eagerly (for comparison)."""

    def __init__(self, model, batch_size: int, max_cache_len: int, use_graph: bool = True):
        from transformers import StaticCache

        self.model = model
        self.device = next(model.parameters()).device
        self.batch_size = batch_size
        self.max_cache_len = max_cache_len
        self.use_graph = use_graph
        self.cache = StaticCache(config=model.config, max_cache_len=max_cache_len)
        self._tok = torch.zeros((batch_size, 1), dtype=torch.long, device=self.device)
        self._pos = torch.zeros((1,), dtype=torch.long, device=self.device)
        self._pos0 = self._pos.view(())  # 0-d view for the cache's write counters
        self._pos_ids = torch.zeros((batch_size, 1), dtype=torch.long, device=self.device)
        self._next = None
        self._logits = None
        self._graph = None

    def _step(self) -> tuple[torch.Tensor, torch.Tensor]:
        # HF's StaticLayer writes at its own device-side counter
        # (cumulative_length) and bumps it in place; pin every layer's counter
        # to the cache position first, so warm-up, capture and replays all
        # write the token at its position (one multi-tensor copy kernel).
        counters = [layer.cumulative_length for layer in self.cache.layers]
        torch._foreach_copy_(counters, [self._pos0] * len(counters))
        out = self.model(input_ids=self._tok, past_key_values=self.cache, cache_position=self._pos,
                         position_ids=self._pos_ids, use_cache=True)
        logits = out.logits[:, -1]
        return logits, logits.argmax(-1, keepdim=True)

    def _capture(self) -> None:
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self._step()  # warm-up: kernel selection and lazy allocations happen outside the capture
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        self._graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self._graph):
            self._logits, self._next = self._step()

    @torch.inference_mode()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int, return_logits: bool = False):
        B, S = input_ids.shape
        if B != self.batch_size:
            raise ValueError(f"batch size {B} != the decoder's {self.batch_size}")
        if S + max_new_tokens > self.max_cache_len:
            raise ValueError(f"{S} + {max_new_tokens} tokens exceed max_cache_len {self.max_cache_len}")
        self.cache.reset()
        pos = torch.arange(S, device=self.device)
        out = self.model(input_ids=input_ids, past_key_values=self.cache, cache_position=pos,
                         position_ids=pos.unsqueeze(0).expand(B, S), use_cache=True)
        logits = out.logits[:, -1]
        tok = logits.argmax(-1, keepdim=True)
        toks = [tok]
        step_logits = [logits.to(torch.float32, copy=True)] if return_logits else None
        for i in range(max_new_tokens - 1):
            self._tok.copy_(tok)
            self._pos.fill_(S + i)
            self._pos_ids.fill_(S + i)
            if not self.use_graph:
                logits, tok = self._step()
            else:
                if self._graph is None:
                    self._capture()
                self._graph.replay()
                logits, tok = self._logits, self._next.clone()
            toks.append(tok)
            if return_logits:
                # a copy: the graph's output buffer is rewritten by the next replay
                step_logits.append(logits.to(torch.float32, copy=True))
        ids = torch.cat([input_ids] + toks, dim=1)
        return (ids, torch.stack(step_logits, dim=1)) if return_logits else ids
