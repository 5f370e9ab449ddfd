"""Paged KV cache: page pools, per-sequence fragment lists, decode over a tile
table, and a prune that frees the dropped span's pages and re-rotates the kept
suffix's keys in place.

threadcut keeps each layer's cache in one growing buffer, so a prune moves the
whole kept suffix C (threadcut/kv.py:28-41, 83-92). Its README
(README.md:141-144) names the next step: with a paged cache, dropping the span
frees pages and C needs only a key re-rotation. This module is that cache:

- Every layer has a K pool and a V pool ``[pages, Hkv, P, D]``. A page holds P
  consecutive token slots of one sequence, and every layer uses the same page
  ids, so one page table serves all of them.
- A sequence is an ordered list of fragments ``(page, first slot, count)``.
  Appends extend the last fragment while its page has room, then take a new
  page. A prune cuts the list at the dropped span. A page no fragment uses any
  more goes back to the free list, and the kept fragments stay where they are.
- Decode reads a tile table: each fragment is cut into tiles of at most 16
  slots, entries ``{page, first slot, rows, 0}``
  (``tc_decode_paged_attention``). Attention over a set of keys does not
  depend on their order, so holes left by prunes cost nothing.
- The prune's only device work is ``tc_paged_rotate_keys``: C's keys rotated
  in place by -(c0 - a) positions with the reference's rotation
  (threadcut/kv.py:20-25), for every layer in one launch. V is not touched.

``PageTable`` is the bookkeeping alone (no device), ``PagedKV`` adds the pools.
"""
import numpy as np
import torch

from . import _lib
from .flash_decode import HEAD_DIM, num_splits
from .kv import rope_table

TILE = 16  # rows per tile-table entry (the decode kernel's tile)


def _cut(frags, lo, hi):
    """The fragments covering logical tokens [lo, hi) of a fragment list."""
    out, pos = [], 0
    for page, start, count in frags:
        a, b = max(lo, pos), min(hi, pos + count)
        if a < b:
            out.append((page, start + a - pos, b - a))
        pos += count
        if pos >= hi:
            break
    return out


def tiles_of(frags):
    """Tile entries (page, first slot, rows) of a fragment list: each fragment
    is cut at multiples of 16 slots, so full tiles are 16-slot aligned."""
    out = []
    for page, start, count in frags:
        s, end = start, start + count
        while s < end:
            e = min(end, (s // TILE + 1) * TILE)
            out.append((page, s, e - s))
            s = e
    return out


class PageTable:
    """Pages of `page_tokens` slots shared by `batch` sequences (host bookkeeping)."""

    def __init__(self, num_pages, page_tokens, batch=1):
        if num_pages < 1 or page_tokens < 1 or batch < 1:
            raise ValueError("PageTable needs num_pages, page_tokens and batch >= 1")
        self.num_pages = int(num_pages)
        self.page_tokens = int(page_tokens)
        self.free = list(range(self.num_pages - 1, -1, -1))  # pop() hands out the lowest id first
        self.frags = [[] for _ in range(batch)]
        self.version = 0  # bumped on every change, so device copies know when to refresh

    @property
    def batch(self):
        return len(self.frags)

    def length(self, b):
        return sum(c for _, _, c in self.frags[b])

    def reserve(self, b, n):
        """Slots (page, slot) for the next n tokens of sequence b, in order."""
        if n < 0:
            raise ValueError("reserve: n must be >= 0")
        fr = self.frags[b]
        need_pages = 0
        room = 0
        if fr:
            page, start, count = fr[-1]
            room = self.page_tokens - (start + count)
        if n > room:
            need_pages = -(-(n - room) // self.page_tokens)
        if need_pages > len(self.free):
            raise RuntimeError(f"PageTable: {need_pages} pages needed, {len(self.free)} free")
        out = []
        while len(out) < n:
            if fr and fr[-1][1] + fr[-1][2] < self.page_tokens:
                page, start, count = fr[-1]
                take = min(n - len(out), self.page_tokens - (start + count))
                out += [(page, start + count + i) for i in range(take)]
                fr[-1] = (page, start, count + take)
            else:
                fr.append((self.free.pop(), 0, 0))
        self.version += 1
        return out

    def prune(self, b, a, c0, c):
        """Keep tokens [0, a) and [c0, c0 + c) of sequence b; returns (the kept
        suffix's fragments, the pages freed)."""
        n = self.length(b)
        if not (0 <= a <= c0 and c >= 0 and c0 + c <= n):
            raise ValueError(f"prune: split (a={a}, c0={c0}, c={c}) outside a sequence of {n} tokens")
        old = self.frags[b]
        suffix = _cut(old, c0, c0 + c)
        new = _cut(old, 0, a) + suffix
        # Adjacent pieces of one page merge back (a == c0 leaves the list as it was).
        merged = []
        for f in new:
            if merged and merged[-1][0] == f[0] and merged[-1][1] + merged[-1][2] == f[1]:
                merged[-1] = (f[0], merged[-1][1], merged[-1][2] + f[2])
            else:
                merged.append(f)
        kept = {p for p, _, _ in merged}
        freed = sorted({p for p, _, _ in old} - kept)
        self.frags[b] = merged
        self.free += sorted(freed, reverse=True)
        self.version += 1
        return suffix, freed

    def release(self, b):
        """Drop sequence b entirely (its pages return to the free list)."""
        self.free += sorted({p for p, _, _ in self.frags[b]}, reverse=True)
        self.frags[b] = []
        self.version += 1

    def token_slots(self, b):
        """(page, slot) of every token of sequence b in logical order."""
        return [(p, s + i) for p, s, c in self.frags[b] for i in range(c)]

    def tile_table(self):
        """int32 [B, max_tiles, 4] and tiles int32 [B] (numpy)."""
        per = [tiles_of(f) for f in self.frags]
        mt = max(1, max(len(t) for t in per))
        tab = np.zeros((self.batch, mt, 4), dtype=np.int32)
        cnt = np.zeros(self.batch, dtype=np.int32)
        for b, ts in enumerate(per):
            if ts:
                tab[b, :len(ts), :3] = np.asarray(ts, dtype=np.int32)
            cnt[b] = len(ts)
        return tab, cnt


class PagedKV:
    """A paged KV cache of `layers` layers on one GPU.

    K/V pools are ``[num_pages, kv_heads, page_tokens, 128]`` per layer (zeroed
    at creation); `page_tokens` should be a multiple of 16 so that full tiles
    are aligned. Sequences grow with `append` and shrink with `prune`.
    """

    def __init__(self, layers, kv_heads, num_pages, page_tokens=64, batch=1, dtype=torch.float16, device="cuda"):
        dev = torch.device(device)
        if dev.type != "cuda":
            raise RuntimeError("PagedKV: the pools must live on a GPU (the kernels are HIP only)")
        if dtype not in (torch.float16, torch.bfloat16):
            raise TypeError(f"PagedKV: dtype {dtype} unsupported (float16, bfloat16)")
        self.table = PageTable(num_pages, page_tokens, batch)
        shape = (num_pages, kv_heads, page_tokens, HEAD_DIM)
        self.k_pools = [torch.zeros(shape, dtype=dtype, device=dev) for _ in range(layers)]
        self.v_pools = [torch.zeros(shape, dtype=dtype, device=dev) for _ in range(layers)]
        self.kv_heads = kv_heads
        self.dtype = dtype
        self.device = dev
        self._dev_table = None  # (version, table, tiles, max_tiles)

    @property
    def layers(self):
        return len(self.k_pools)

    def length(self, b=0):
        return self.table.length(b)

    def _strides(self):
        return _lib.i64x3(*self.k_pools[0].stride()[:3])

    def append(self, b, ks, vs):
        """Append tokens to sequence b: ks/vs are per-layer [Hkv, n, D] (or
        [1, Hkv, n, D]) tensors on the pools' device."""
        if len(ks) != self.layers or len(vs) != self.layers:
            raise ValueError(f"append: {self.layers} layers of K and V expected")
        n = ks[0].shape[-2]
        slots = self.table.reserve(b, n)
        if n == 0:
            return
        idx = torch.tensor(slots, dtype=torch.long).to(self.device)
        pages, sl = idx[:, 0], idx[:, 1]
        for kp, vp, k, v in zip(self.k_pools, self.v_pools, ks, vs):
            k = k.reshape(self.kv_heads, n, HEAD_DIM)
            v = v.reshape(self.kv_heads, n, HEAD_DIM)
            kp[pages, :, sl] = k.transpose(0, 1).to(self.dtype)
            vp[pages, :, sl] = v.transpose(0, 1).to(self.dtype)

    def gather(self, layer, b=0):
        """Sequence b's K and V of one layer in logical order, [Hkv, n, D] copies."""
        slots = self.table.token_slots(b)
        if not slots:
            z = torch.empty(self.kv_heads, 0, HEAD_DIM, dtype=self.dtype, device=self.device)
            return z, z.clone()
        idx = torch.tensor(slots, dtype=torch.long).to(self.device)
        k = self.k_pools[layer][idx[:, 0], :, idx[:, 1]].transpose(0, 1).contiguous()
        v = self.v_pools[layer][idx[:, 0], :, idx[:, 1]].transpose(0, 1).contiguous()
        return k, v

    def device_table(self):
        """(tile table int32 [B, max_tiles, 4], tiles int32 [B], max_tiles) on the device."""
        ver = self.table.version
        if self._dev_table is None or self._dev_table[0] != ver:
            tab, cnt = self.table.tile_table()
            self._dev_table = (ver, torch.from_numpy(tab).to(self.device), torch.from_numpy(cnt).to(self.device),
                               tab.shape[1])
        return self._dev_table[1:]

    def decode(self, layer, q, scale, out=None, split=None):
        """softmax(q·Kᵀ·scale)·V over each sequence's keys of one layer.

        q [B, Hkv, G, D] (G query heads per KV head, last dim contiguous) in the
        pools' dtype; returns out [B, Hkv, G, D]. Enqueued on the current stream.
        """
        _lib.require_gpu(q, what="PagedKV.decode")
        b, hkv, g, d = q.shape
        if b != self.table.batch or hkv != self.kv_heads or d != HEAD_DIM or q.dtype != self.dtype:
            raise ValueError(f"PagedKV.decode: q {tuple(q.shape)} {q.dtype} does not fit the cache")
        if q.stride(3) != 1:
            raise ValueError("PagedKV.decode: q must have a contiguous last dimension")
        if out is None:
            out = torch.empty_like(q)
        tab, cnt, mt = self.device_table()
        lib = _lib.load()
        kp, vp = self.k_pools[layer], self.v_pools[layer]
        with torch.cuda.device(q.device):
            s = num_splits(b, hkv, TILE * mt, split, ragged=b > 1)
            nbytes = lib.tc_decode_workspace_bytes(b, hkv, g, d, s)
            ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=q.device)
            rc = lib.tc_decode_paged_attention(
                q.data_ptr(), _lib.i64x3(*q.stride()[:3]), kp.data_ptr(), vp.data_ptr(), self._strides(),
                kp.shape[0], kp.shape[2], tab.data_ptr(), cnt.data_ptr(), mt, b, hkv, g, d,
                _lib.dtype_code(self.dtype), float(scale), int(split or 0), ws.data_ptr(), ws.numel(),
                out.data_ptr(), _lib.i64x3(*out.stride()[:3]), _lib.stream_of(q.device))
            _lib.check(rc, "tc_decode_paged_attention")
        return out

    def prune(self, b, s, inv_freq):
        """Keep tokens [0, s.a) and [s.c0, s.c0 + s.c) of sequence b (a threadcut
        Split): the dropped span's pages are freed and the kept suffix's keys are
        re-rotated in place by -(c0 - a) positions in every layer. Returns the
        freed page ids."""
        suffix, freed = self.table.prune(b, s.a, s.c0, s.c)
        gap = s.c0 - s.a
        tiles = tiles_of(suffix)
        if gap and tiles:
            t = np.zeros((len(tiles), 4), dtype=np.int32)
            t[:, :3] = np.asarray(tiles, dtype=np.int32)
            td = torch.from_numpy(t).to(self.device)
            table = _lib.float_array(rope_table(-gap, inv_freq))
            lib = _lib.load()
            kp = _lib.ptr_array([p.data_ptr() for p in self.k_pools])
            with torch.cuda.device(self.device):
                rc = lib.tc_paged_rotate_keys(kp, self.layers, self._strides(), self.k_pools[0].shape[0],
                                              self.k_pools[0].shape[2], td.data_ptr(), len(tiles), self.kv_heads,
                                              HEAD_DIM, _lib.dtype_code(self.dtype), table,
                                              _lib.stream_of(self.device))
                _lib.check(rc, "tc_paged_rotate_keys")
        return freed
