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

The host keeps each layer's token count in step (``n``) so that the cache is
an ordinary cache again after ``close()``: splice, prefill and eager decode
work on it as before.

The model must run the "threadcut" attention: each layer's new K/V row is
written by its decode kernel, and another attention would read the row
unwritten, so DecodeGraph refuses a model set to any other.

Two cache kinds are captured: ``kv.new_cache`` caches (GrowingLayer buffers,
grown once to the step's capacity; the append position is a device counter)
and ``paged.new_paged_cache`` caches (slots for the new tokens reserved ahead
in the page table, whose tile table and token offsets are uploaded once; the
sequence lengths are the device counter).
"""
import torch

from . import attention, kv, paged


class _GrowingCache:
    """The GrowingLayer cache of a DecodeGraph."""

    def __init__(self, cache, batch, max_new_tokens):
        layers = cache.layers
        if not layers or not all(isinstance(l, kv.GrowingLayer) and getattr(l, "kbuf", None) is not None
                                 for l in layers):
            raise ValueError("DecodeGraph: needs a prefilled kv.new_cache() or paged.new_paged_cache() cache")
        n = layers[0].n
        if any(l.n != n for l in layers):
            raise ValueError("DecodeGraph: every layer must hold the same number of tokens")
        if layers[0].kbuf.shape[0] != batch:
            raise ValueError(f"DecodeGraph: cache batch {layers[0].kbuf.shape[0]} != {batch}")
        self.layers = layers
        for l in layers:
            l.flush()
            l._reserve(n + max_new_tokens + 1, l.kbuf)
            l._view()
        self.device = layers[0].kbuf.device
        self.capacity = layers[0].kbuf.shape[-2]
        # The captured kernels hold these buffers' addresses: keep the tensors, and check
        # before every replay that each layer still uses them.
        self.buffers = [(l.kbuf, l.vbuf) for l in layers]

    def attach(self, pos):
        for l in self.layers:
            l.device_pos = pos

    def in_step(self, flag):
        for l in self.layers:
            l.in_graph_step = flag

    def advance(self, k):
        for l in self.layers:
            l.n += k
            l._view()

    def unchanged(self, n, pos):
        return all(l.kbuf is kb and l.vbuf is vb and l.n == n and l.device_pos is pos
                   for l, (kb, vb) in zip(self.layers, self.buffers))

    def detach(self):
        for l in self.layers:
            l.device_pos = None
            l.pending = None
            l._view()


class _PagedCache:
    """The paged cache of a DecodeGraph: max_new_tokens + 1 slots per sequence reserved in
    the page table up front, the tables uploaded once, the unused slots released on close."""

    def __init__(self, cache, batch, max_new_tokens):
        self.state = state = paged.state_of(cache)
        if state.kv is None:
            raise ValueError("DecodeGraph: the paged cache holds no tokens yet")
        table = state.kv.table
        self.layers = layers = cache.layers
        for l in layers:
            l.flush()
        n = layers[0].n
        if any(l.n != n for l in layers) or any(table.length(b) != n for b in range(table.batch)):
            raise ValueError("DecodeGraph: every layer and sequence of the paged cache must hold the same tokens")
        if table.batch != batch:
            raise ValueError(f"DecodeGraph: cache batch {table.batch} != {batch}")
        for b in range(batch):
            table.reserve(b, max_new_tokens + 1)
        self.device = state.kv.device
        self.capacity = n + max_new_tokens + 1
        # Uploaded once here; the captured kernels read these tensors on every replay.
        self.tables = (state.kv.device_table(), state.kv.device_offsets())
        self.version = table.version

    def attach(self, pos):
        self.state.device_lens = pos

    def in_step(self, flag):
        self.state.in_graph_step = flag

    def advance(self, k):
        for l in self.layers:
            l.n += k

    def unchanged(self, n, pos):
        return (self.state.kv.table.version == self.version and self.state.device_lens is pos
                and all(l.n == n for l in self.layers))

    def detach(self):
        self.state.device_lens = None
        for l in self.layers:
            l.pending = None
        n = self.layers[0].n
        table = self.state.kv.table
        for b in range(table.batch):
            table.prune(b, n, table.length(b), 0)


class DecodeGraph:
    """Captured decode step of `model` (run with the "threadcut" attention) over `cache`.

    cache: a prefilled ``kv.new_cache`` or ``paged.new_paged_cache`` cache
    (every layer holding the same n tokens), with room made once for
    `max_new_tokens` more; then the step is captured. ``step(ids)`` feeds one
    token per sequence and returns the logits [B, vocab] of that position (a
    static tensor, overwritten by the next step). ``close()`` hands the cache
    back.
    """

    def __init__(self, model, cache, max_new_tokens, batch=1):
        types = set(getattr(model.config, "layer_types", None) or ["full_attention"])
        if types != {"full_attention"}:
            raise ValueError(f"DecodeGraph: layer types {sorted(types)}; only full-attention models are captured")
        impl = getattr(model.config, "_attn_implementation", None)
        if impl != attention.NAME:
            # The captured step leaves each layer's new K/V row to the attention kernel,
            # which writes it while it attends; any other attention would read a stale row.
            raise ValueError(f"DecodeGraph: the model runs the {impl!r} attention; call "
                             f"model.set_attn_implementation({attention.NAME!r}) first")
        self.store = (_PagedCache if paged.state_of(cache) is not None else _GrowingCache)(cache, batch,
                                                                                          max_new_tokens)
        dev = self.store.device
        self.model, self.cache, self.layers, self.batch = model, cache, cache.layers, batch
        self.capacity = self.store.capacity
        n = self.layers[0].n
        self.pos = torch.full((batch,), n, dtype=torch.int32, device=dev)
        self.position_ids = torch.full((batch, 1), n, dtype=torch.long, device=dev)
        self.ids = torch.zeros((batch, 1), dtype=torch.long, device=dev)
        self.store.attach(self.pos)

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
        self.store.advance(-1)

    @torch.no_grad()
    def _step_body(self):
        # One new token per sequence sees every cached token: no mask. Handing the
        # (empty) mask mapping over keeps transformers from building a mask tensor,
        # which it does while a graph is being captured.
        self.store.in_step(True)
        try:
            out = self.model(input_ids=self.ids, position_ids=self.position_ids, past_key_values=self.cache,
                             attention_mask={"full_attention": None}, use_cache=True, logits_to_keep=1)
        finally:
            self.store.in_step(False)
        logits = out.logits[:, -1]
        self.pos.add_(1)
        self.position_ids.add_(1)
        return logits

    def _rewind(self):
        self.pos.sub_(1)
        self.position_ids.sub_(1)
        self.store.advance(-1)

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
        if not self.store.unchanged(n, self.pos):
            raise RuntimeError("DecodeGraph: the cache changed outside the graph since capture")
        self.ids.copy_(torch.as_tensor(ids).reshape(self.batch, 1), non_blocking=True)
        self.graph.replay()
        self.store.advance(1)
        return self.logits

    def close(self):
        """Return the layers to host-counted operation (views refreshed, reserved slots freed)."""
        if self.graph is None:
            return
        torch.cuda.current_stream(self.pos.device).synchronize()
        self.store.detach()
        self.graph = None
