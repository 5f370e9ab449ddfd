"""KV cache surgery on MI355X: drop a pruned span B and move C left, keys re-rotated.

Drop-in for threadcut/kv.py:15-98. Keys are cached after RoPE and rotations
compose, so rotating a key stored at position p by -gap gives the key at
p - gap; values carry no position and move unchanged. The per-layer torch op
chains of the reference (about eight kernels and fp32 temporaries per layer,
36 layers) become one HIP launch (``tc_splice_rope``) that gathers, rotates
and stores every layer's suffix in place. Tensors the kernels do not take
(host tensors, float32, head_dim other than 128) keep the reference's own
torch op sequence, which is what the reference runs for them.

The rotation table cos/sin(delta * inv_freq) is built on the host with the
reference's own op order (threadcut/kv.py:22-23) and passed by value in the
kernel arguments; the kernel then evaluates fl(k*cos) + fl(rotate_half(k)*sin)
without contraction, so shifted keys match the reference's fp32 op sequence
bit for bit.
"""
import torch
from transformers import DynamicCache
from transformers.cache_utils import DynamicLayer

from . import _lib
from .match import Split  # noqa: F401  (re-exported: the splice contract)

HEAD_DIM = 128

# Deferred single-token appends of GrowingLayers in fused-append mode, by the
# address of the layer's K buffer; the "threadcut" attention takes them.
_PENDING = {}


def take_pending(key):
    """The GrowingLayer whose deferred append `key` (a [..., :n, :] view) carries, or None.

    Clears the registration; the caller must then write the new token itself
    (flash_decode.decode_append_into does, inside the attention kernel).
    """
    if not key.is_cuda:
        return None
    layer = _PENDING.get(key.data_ptr())
    if layer is None or layer.pending is None or key.shape[-2] != layer.n:
        return None
    del _PENDING[key.data_ptr()]
    return layer


def rotate_half(x):
    """cat(-x2, x1) over the two halves of the last dim (threadcut/kv.py:15-17)."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def rope_table(delta, inv_freq):
    """Host fp32 [D] = cos(angle) ++ sin(angle), angle = delta * inv_freq.

    Same op sequence as threadcut/kv.py:22-23 (`delta * inv_freq.float()`,
    emb = cat(angle, angle), emb.cos(), emb.sin()), evaluated on the host CPU;
    emb's upper half repeats the lower one, so only the lower half is kept.
    """
    f = inv_freq.detach().to("cpu").float()
    angle = delta * f
    emb = torch.cat((angle, angle))
    half = f.numel()
    return torch.cat((emb.cos()[:half], emb.sin()[:half]))


def _hip_ok(t):
    """True if the HIP splice kernels take this cache tensor."""
    return t.is_cuda and t.dtype in _lib.DTYPES and t.shape[-1] == HEAD_DIM and t.stride(-1) == 1


def _shift_keys_torch(keys, delta, inv_freq):
    """The reference's rotation in torch ops (threadcut/kv.py:20-25): fp32 math on the
    keys' device, k*cos + rotate_half(k)*sin, cast back to the keys' dtype."""
    table = rope_table(delta, inv_freq).to(keys.device)
    half = table.numel() // 2
    cos = torch.cat((table[:half], table[:half]))
    sin = torch.cat((table[half:], table[half:]))
    k = keys.float()
    return (k * cos + rotate_half(k) * sin).to(keys.dtype)


def _splice_layer_torch(kbuf, vbuf, s, inv_freq):
    """GrowingLayer.splice of the reference (threadcut/kv.py:83-92) on one layer's buffers:
    C read out (keys rotated by -gap, or copied when gap is 0), then written at a."""
    if s.c:
        k = kbuf[..., s.c0:s.c0 + s.c, :]
        k = _shift_keys_torch(k, -s.gap, inv_freq) if s.gap else k.clone()
        v = vbuf[..., s.c0:s.c0 + s.c, :].clone()
        kbuf[..., s.a:s.a + s.c, :] = k
        vbuf[..., s.a:s.a + s.c, :] = v


def _as4(t):
    if t.dim() == 4:
        return t
    if t.dim() == 3:
        return t.unsqueeze(0)
    if t.dim() == 2:
        return t.unsqueeze(0).unsqueeze(0)
    raise ValueError(f"expected a [..., tokens, head_dim] tensor of rank 2-4, got {tuple(t.shape)}")


def shift_keys(keys, delta, inv_freq):
    """Move post-RoPE keys by `delta` positions (negative = left); new tensor.

    threadcut/kv.py:20-25: fp32 math, result in keys.dtype. A [..., tokens, 128]
    fp16/bf16 GPU tensor with a contiguous last dim runs the HIP kernel; other
    keys (host tensors, float32, other head dims) the reference's torch ops.
    """
    if not _hip_ok(keys):
        return _shift_keys_torch(keys, delta, inv_freq)
    k4 = _as4(keys)
    b, h, t, d = k4.shape
    if d != HEAD_DIM:
        raise ValueError(f"shift_keys: head_dim {d} unsupported (128)")
    if k4.stride(3) != 1:
        raise ValueError("shift_keys: keys must have a contiguous last dimension")
    out = torch.empty(keys.shape, dtype=keys.dtype, device=keys.device)
    o4 = _as4(out)
    table = _lib.float_array(rope_table(delta, inv_freq))
    lib = _lib.load()
    with torch.cuda.device(keys.device):
        rc = lib.tc_shift_keys(k4.data_ptr(), _lib.i64x3(k4.stride(0), k4.stride(1), k4.stride(2)),
                               o4.data_ptr(), _lib.i64x3(o4.stride(0), o4.stride(1), o4.stride(2)),
                               b, h, t, d, _lib.dtype_code(keys.dtype), table, _lib.stream_of(keys.device))
    _lib.check(rc, "tc_shift_keys")
    return out


def _splice_buffers(kbufs, vbufs, s, inv_freq):
    """In-place A·B·C -> A·C over equally shaped [B, H, cap, 128] buffers."""
    k0 = kbufs[0]
    b, h, cap, d = k0.shape
    for t in (*kbufs, *vbufs):
        if t.shape != k0.shape or t.stride() != k0.stride() or t.dtype != k0.dtype or t.device != k0.device:
            raise ValueError("splice: every layer's K/V buffer must share shape, strides, dtype and device")
    _lib.require_gpu(k0, what="splice")
    table = _lib.float_array(rope_table(-s.gap, inv_freq)) if s.c and s.gap else None
    lib = _lib.load()
    with torch.cuda.device(k0.device):
        rc = lib.tc_splice_rope(_lib.ptr_array([t.data_ptr() for t in kbufs]),
                                _lib.ptr_array([t.data_ptr() for t in vbufs]), len(kbufs),
                                _lib.i64x3(k0.stride(0), k0.stride(1), k0.stride(2)), b, h, cap, d,
                                _lib.dtype_code(k0.dtype), s.a, s.c0, s.c, table, _lib.stream_of(k0.device))
    _lib.check(rc, "tc_splice_rope")


def _group_by_layout(layers):
    groups = {}
    for layer in layers:
        t = layer.kbuf
        key = (tuple(t.shape), t.stride(), t.dtype, t.device)
        groups.setdefault(key, []).append(layer)
    return groups.values()


def splice(cache, s, inv_freq):
    """Rewrite every layer of a DynamicCache from A·B·C·(tail) to A·C (threadcut/kv.py:28-41).

    A paged cache (paged.new_paged_cache) is pruned instead: the pages of the dropped span
    go back to the free list and the kept suffix's keys are re-rotated where they are."""
    from . import paged

    state = paged.state_of(cache)
    if state is not None:
        state.check_not_captured("splice")
        for layer in cache.layers:
            layer.flush()
        if state.kv is not None:
            for b in range(state.batch):
                state.kv.prune(b, s, inv_freq)
        for layer in cache.layers:
            layer.n = s.a + s.c
        return
    if all(isinstance(layer, GrowingLayer) for layer in cache.layers):
        live = [layer for layer in cache.layers if getattr(layer, "kbuf", None) is not None]
        for layer in live:
            layer._check_not_captured("splice")
        for layer in live:
            layer.flush()
        for layer in live:
            if s.c0 + s.c > layer.n:
                raise ValueError(f"splice: suffix [{s.c0}, {s.c0 + s.c}) past the {layer.n} cached tokens")
        if s.c and s.gap:
            for group in _group_by_layout(live):
                if _hip_ok(group[0].kbuf):
                    _splice_buffers([l.kbuf for l in group], [l.vbuf for l in group], s, inv_freq)
                else:
                    for l in group:
                        _splice_layer_torch(l.kbuf, l.vbuf, s, inv_freq)
        for layer in live:
            layer.n = s.a + s.c
            layer._view()
        return
    layers = cache.layers
    k0 = layers[0].keys
    if not all(_hip_ok(t) for l in layers for t in (l.keys, l.values)):
        _splice_index_select_torch(layers, s, inv_freq)
        return
    b, h, n, d = k0.shape
    if s.c0 + s.c > n or s.a > n:
        raise ValueError(f"splice: split {s} past the {n} cached tokens")
    new_k = [torch.empty((b, h, s.a + s.c, d), dtype=k0.dtype, device=k0.device) for _ in layers]
    new_v = [torch.empty_like(t) for t in new_k]
    for layer in layers:
        for t in (layer.keys, layer.values):
            if t.shape != k0.shape or t.stride() != k0.stride() or t.dtype != k0.dtype:
                raise ValueError("splice: every layer's keys/values must share shape, strides and dtype")
    table = _lib.float_array(rope_table(-s.gap, inv_freq)) if s.c and s.gap else None
    src_st = _lib.i64x3(k0.stride(0), k0.stride(1), k0.stride(2))
    t0 = new_k[0]
    dst_st = _lib.i64x3(t0.stride(0), t0.stride(1), t0.stride(2))
    lib = _lib.load()
    with torch.cuda.device(k0.device):
        rc = lib.tc_splice_copy(_lib.ptr_array([l.keys.data_ptr() for l in layers]),
                                _lib.ptr_array([l.values.data_ptr() for l in layers]), src_st, n,
                                _lib.ptr_array([t.data_ptr() for t in new_k]),
                                _lib.ptr_array([t.data_ptr() for t in new_v]), dst_st, len(layers),
                                b, h, d, _lib.dtype_code(k0.dtype), s.a, s.c0, s.c, table,
                                _lib.stream_of(k0.device))
    _lib.check(rc, "tc_splice_copy")
    for layer, k, v in zip(layers, new_k, new_v):
        layer.keys, layer.values = k, v


def _splice_index_select_torch(layers, s, inv_freq):
    """The reference's splice of plain DynamicLayers (threadcut/kv.py:34-41) in torch ops:
    keep [0, a) and [c0, c0 + c), then rotate the kept suffix's keys by -gap."""
    n = layers[0].keys.shape[-2]
    if s.c0 + s.c > n or s.a > n:
        raise ValueError(f"splice: split {s} past the {n} cached tokens")
    device = layers[0].keys.device
    keep = torch.cat((torch.arange(0, s.a), torch.arange(s.c0, s.c0 + s.c))).to(device)
    for layer in layers:
        k = layer.keys.index_select(2, keep)
        v = layer.values.index_select(2, keep)
        if s.c and s.gap:
            k[:, :, s.a:] = _shift_keys_torch(k[:, :, s.a:], -s.gap, inv_freq)
        layer.keys, layer.values = k, v


class KVSlab:
    """One allocation [L, 2, B, Hkv, cap, D] holding every layer's K and V buffers.

    Layer l's buffers are the views ``slab[l, 0]`` and ``slab[l, 1]``, each a
    contiguous [B, Hkv, cap, D] tensor like a GrowingLayer's own, so kernels,
    the splice's pointer table and the engine's ``layer.keys`` views see the
    same layout. Capacity grows for all layers at once (the GrowingLayer rule,
    max(need, 1.25 cap, cap + 2048)), with one copy of each layer's tokens.
    """

    def __init__(self, layers):
        self.layers = layers
        self.tensor = None

    @property
    def capacity(self):
        return 0 if self.tensor is None else self.tensor.shape[-2]

    def reserve(self, need, like):
        """Grow to hold `need` tokens per layer (like: a [B, Hkv, *, D] tensor of the cache's type)."""
        cap = self.capacity
        if need <= cap:
            return
        for layer in self.layers:
            if getattr(layer, "kbuf", None) is not None:
                layer.flush()
        new = max(need, int(cap * 1.25), cap + 2048)
        b, h, d = like.shape[0], like.shape[1], like.shape[-1]
        t = like.new_empty((len(self.layers), 2, b, h, new, d))
        for i, layer in enumerate(self.layers):
            n = getattr(layer, "n", 0) if getattr(layer, "kbuf", None) is not None else 0
            if n:
                t[i, 0, :, :, :n] = layer.kbuf[..., :n, :]
                t[i, 1, :, :, :n] = layer.vbuf[..., :n, :]
        self.tensor = t
        for i, layer in enumerate(self.layers):
            if getattr(layer, "kbuf", None) is not None:
                layer.kbuf, layer.vbuf = t[i, 0], t[i, 1]
                layer._view()


class GrowingLayer(DynamicLayer):
    """DynamicLayer backed by a preallocated buffer (threadcut/kv.py:44-92).

    Appending a token writes in place instead of re-copying the cache with
    torch.cat. Capacity grows by max(need, 1.25 * cap, cap + 2048) tokens.
    ``keys``/``values`` are views ``kbuf[..., :n, :]``.

    With ``fused_append`` (for models run with the "threadcut" attention), a
    single-token GPU update does not copy: the new rows stay pending and the
    decode attention kernel writes them while it attends. Any other access
    path (a later update, splice, crop) writes a pending row first.
    """

    fused_append = False
    pending = None
    # Set by new_cache(slab=True): the shared KVSlab and this layer's index in it.
    slab = None
    slab_index = 0
    # Set by graph.DecodeGraph: an int32 [B] device tensor holding the token
    # count, so the decode kernel takes the append position from the device
    # (tc_decode_append_attention_at) instead of from the host-side n.
    device_pos = None
    # True while graph.DecodeGraph runs its own step body (warm-up, capture).
    in_graph_step = False

    def _check_not_captured(self, what):
        """A layer held by a live DecodeGraph changes only through the graph's step:
        anything else would leave the captured kernels writing stale positions or
        freed buffers."""
        if self.device_pos is not None and not self.in_graph_step:
            raise RuntimeError(f"GrowingLayer.{what}: a DecodeGraph holds this cache; close() it first")

    def lazy_initialization(self, key_states, value_states):
        super().lazy_initialization(key_states, value_states)
        self.n, self.kbuf, self.vbuf = 0, None, None

    def flush(self):
        """Write a deferred append that no attention call consumed."""
        if self.pending is not None:
            _PENDING.pop(self.kbuf.data_ptr(), None)
            k, v = self.pending
            self.kbuf[..., self.n - 1:self.n, :] = k
            self.vbuf[..., self.n - 1:self.n, :] = v
            self.pending = None

    def _reserve(self, need, like):
        if self.slab is not None:
            self.slab.reserve(need, like)
            if self.kbuf is None:
                t = self.slab.tensor
                self.kbuf, self.vbuf = t[self.slab_index, 0], t[self.slab_index, 1]
            return
        cap = 0 if self.kbuf is None else self.kbuf.shape[-2]
        if need <= cap:
            return
        new = max(need, int(cap * 1.25), cap + 2048)
        kb = like.new_empty((*like.shape[:-2], new, like.shape[-1]))
        vb = torch.empty_like(kb)
        if self.n:
            kb[..., :self.n, :] = self.kbuf[..., :self.n, :]
            vb[..., :self.n, :] = self.vbuf[..., :self.n, :]
        self.kbuf, self.vbuf = kb, vb

    def _view(self):
        self.keys, self.values = self.kbuf[..., :self.n, :], self.vbuf[..., :self.n, :]

    def update(self, key_states, value_states, *args, **kwargs):
        self._check_not_captured("update")
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        self.flush()
        add = key_states.shape[-2]
        self._reserve(self.n + add, key_states)
        if (self.fused_append or self.device_pos is not None) and add == 1 and key_states.is_cuda:
            self.pending = (key_states, value_states)
            _PENDING[self.kbuf.data_ptr()] = self
        else:
            self.kbuf[..., self.n:self.n + add, :] = key_states
            self.vbuf[..., self.n:self.n + add, :] = value_states
        self.n += add
        self._view()
        return self.keys, self.values

    def crop(self, max_length):
        self._check_not_captured("crop")
        self.flush()
        self.n = min(self.n, max_length)
        self._view()

    def splice(self, s, inv_freq):
        """In-place A·B·C -> A·C: only C is touched, so a prune costs O(|C|)."""
        self._check_not_captured("splice")
        self.flush()
        if s.c0 + s.c > self.n:
            raise ValueError(f"splice: suffix [{s.c0}, {s.c0 + s.c}) past the {self.n} cached tokens")
        if s.c and s.gap:
            if _hip_ok(self.kbuf):
                _splice_buffers([self.kbuf], [self.vbuf], s, inv_freq)
            else:
                _splice_layer_torch(self.kbuf, self.vbuf, s, inv_freq)
        self.n = s.a + s.c
        self._view()


def new_cache(config, fused_append=False, slab=False):
    """A DynamicCache whose layers are GrowingLayers (threadcut/kv.py:95-98).

    fused_append=True defers single-token appends into the decode attention
    kernel; use it only with the "threadcut" attention implementation.
    slab=True keeps every layer's buffers in one [L, 2, B, Hkv, cap, D]
    allocation (KVSlab) that grows for all layers at once.
    """
    cache = DynamicCache(config=config)
    cache.layers = [GrowingLayer() for _ in cache.layers]
    shared = KVSlab(cache.layers) if slab else None
    for i, layer in enumerate(cache.layers):
        layer.fused_append = fused_append
        layer.slab, layer.slab_index = shared, i
    return cache
