"""The decode step as one HIP graph (the per-token loop of threadcut/engine.py:88-95).

The reference decodes token by token in eager mode: every step launches the
whole model from Python (36 layers, each a dozen kernels, plus the cache
appends), so at batch 1 the GPU waits on the host between kernels. Here the
step is captured once and replayed per token:

- token ids and position ids enter through static device buffers;
- each layer's cache append and attention is one kernel
  (``tc_decode_append_attention_at``) that takes the append position from a
  device counter shared by the layers, not from a host integer baked into
  the graph;
- the graph ends by advancing that counter and the position ids, so replay
  k writes token n + k and attends over n + k + 1 tokens;
- the logits land in a static buffer.

A decode step of one token per sequence attends to every cached token, so
the step passes transformers an already-prepared empty mask mapping: left to
itself, transformers builds a mask tensor while a graph is being captured
(and the attention call would then take the prefill branch).

The host keeps each GrowingLayer's token count in step (``n``) so that the
cache is an ordinary GrowingLayer cache again after ``close()``: splice,
prefill and eager decode work on it as before.
"""
import torch

from . import kv


class DecodeGraph:
    """Captured decode step of `model` (run with the "threadcut" attention) over `cache`.

    cache: a ``kv.new_cache`` cache that has been prefilled (every layer holds
    the same n tokens). Its buffers are grown once to hold `max_new_tokens`
    more, then the step is captured. ``step(ids)`` feeds one token per
    sequence and returns the logits [B, vocab] of that position (a static
    tensor, overwritten by the next step). ``close()`` hands the cache back.
    """

    def __init__(self, model, cache, max_new_tokens, batch=1):
        layers = cache.layers
        if not layers or not all(isinstance(l, kv.GrowingLayer) and getattr(l, "kbuf", None) is not None
                                 for l in layers):
            raise ValueError("DecodeGraph: needs a prefilled kv.new_cache() cache")
        n = layers[0].n
        if any(l.n != n for l in layers):
            raise ValueError("DecodeGraph: every layer must hold the same number of tokens")
        if layers[0].kbuf.shape[0] != batch:
            raise ValueError(f"DecodeGraph: cache batch {layers[0].kbuf.shape[0]} != {batch}")
        types = set(getattr(model.config, "layer_types", None) or ["full_attention"])
        if types != {"full_attention"}:
            raise ValueError(f"DecodeGraph: layer types {sorted(types)}; only full-attention models are captured")
        dev = layers[0].kbuf.device
        self.model, self.cache, self.layers, self.batch = model, cache, layers, batch
        for l in layers:
            l.flush()
            l._reserve(n + max_new_tokens + 1, l.kbuf)
            l._view()
        self.capacity = layers[0].kbuf.shape[-2]
        # The captured kernels hold these buffers' addresses: keep the tensors, and check
        # before every replay that each layer still uses them.
        self.buffers = [(l.kbuf, l.vbuf) for l in layers]
        self.pos = torch.full((batch,), n, dtype=torch.int32, device=dev)
        self.position_ids = torch.full((batch, 1), n, dtype=torch.long, device=dev)
        self.ids = torch.zeros((batch, 1), dtype=torch.long, device=dev)
        for l in layers:
            l.device_pos = self.pos

        # Warm-up on a side stream (library loading, allocator pools), then undo its token.
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            self._step_body()
        torch.cuda.current_stream(dev).wait_stream(side)
        self._rewind()

        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = self._step_body()
        # Capture ran the Python once and no kernel: take back the host-side count.
        for l in self.layers:
            l.n -= 1

    @torch.no_grad()
    def _step_body(self):
        # One new token per sequence sees every cached token: no mask. Handing the
        # (empty) mask mapping over keeps transformers from building a mask tensor,
        # which it does while a graph is being captured.
        for l in self.layers:
            l.in_graph_step = True
        try:
            out = self.model(input_ids=self.ids, position_ids=self.position_ids, past_key_values=self.cache,
                             attention_mask={"full_attention": None}, use_cache=True, logits_to_keep=1)
        finally:
            for l in self.layers:
                l.in_graph_step = False
        logits = out.logits[:, -1]
        self.pos.add_(1)
        self.position_ids.add_(1)
        return logits

    def _rewind(self):
        self.pos.sub_(1)
        self.position_ids.sub_(1)
        for l in self.layers:
            l.n -= 1
            l._view()

    @property
    def n(self):
        """Tokens in the cache (host-side count)."""
        return self.layers[0].n

    def step(self, ids):
        """Feed token ids [B] (or [B, 1], device or host) and return the logits [B, vocab]."""
        if self.graph is None:
            raise RuntimeError("DecodeGraph: closed")
        n = self.layers[0].n
        if n + 1 > self.capacity:
            raise RuntimeError(f"DecodeGraph: the cache holds {self.capacity} tokens; close() and grow it")
        for l, (kb, vb) in zip(self.layers, self.buffers):
            if l.kbuf is not kb or l.vbuf is not vb or l.n != n or l.device_pos is not self.pos:
                raise RuntimeError("DecodeGraph: the cache changed outside the graph since capture")
        self.ids.copy_(torch.as_tensor(ids).reshape(self.batch, 1), non_blocking=True)
        self.graph.replay()
        for l in self.layers:
            l.n += 1
        return self.logits

    def close(self):
        """Return the layers to host-counted operation (views refreshed)."""
        torch.cuda.current_stream(self.pos.device).synchronize()
        for l in self.layers:
            l.device_pos = None
            l.pending = None
            l._view()
        self.graph = None
