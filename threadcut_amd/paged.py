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


_EMPTY = np.zeros((0, 3), dtype=np.int64)


def _cut(frags, lo, hi):
    """The fragments (rows of an int64 [F, 3] array) covering logical tokens [lo, hi)."""
    if hi <= lo or len(frags) == 0:
        return _EMPTY
    ends = np.cumsum(frags[:, 2])
    begins = ends - frags[:, 2]
    i0 = int(np.searchsorted(ends, lo, side="right"))
    i1 = int(np.searchsorted(begins, hi, side="left"))
    sub = frags[i0:i1].copy()
    if len(sub):
        skip = lo - begins[i0]
        if skip > 0:
            sub[0, 1] += skip
            sub[0, 2] -= skip
        over = ends[i1 - 1] - hi
        if over > 0:
            sub[-1, 2] -= over
        sub = sub[sub[:, 2] > 0]
    return sub


def tiles_of(frags):
    """Tile entries (page, first slot, rows) of a fragment array, int32 [T, 3]:
    each fragment is cut at multiples of 16 slots, so full tiles are 16-slot
    aligned."""
    frags = np.asarray(frags, dtype=np.int64).reshape(-1, 3)
    if len(frags) == 0:
        return np.zeros((0, 3), dtype=np.int32)
    start, end = frags[:, 1], frags[:, 1] + frags[:, 2]
    t0 = start // TILE
    nt = (end - 1) // TILE + 1 - t0
    rep = np.repeat(np.arange(len(frags)), nt)
    k = np.arange(int(nt.sum())) - np.repeat(np.cumsum(nt) - nt, nt)
    lo = np.maximum(start[rep], (t0[rep] + k) * TILE)
    hi = np.minimum(end[rep], (t0[rep] + k + 1) * TILE)
    return np.stack([frags[rep, 0], lo, hi - lo], axis=1).astype(np.int32)


class PageTable:
    """Pages of `page_tokens` slots shared by `batch` sequences (host bookkeeping).

    frags[b] is sequence b's int64 [F, 3] array of (page, first slot, count).
    """

    def __init__(self, num_pages, page_tokens, batch=1):
        if num_pages < 1 or page_tokens < 1 or batch < 1:
            raise ValueError("PageTable needs num_pages, page_tokens and batch >= 1")
        self.num_pages = int(num_pages)
        self.page_tokens = int(page_tokens)
        self.free = list(range(self.num_pages - 1, -1, -1))  # pop() hands out the lowest id first
        self.frags = [_EMPTY.copy() for _ in range(batch)]
        self.version = 0  # bumped on every change, so device copies know when to refresh

    @property
    def batch(self):
        return len(self.frags)

    def length(self, b):
        return int(self.frags[b][:, 2].sum())

    def reserve(self, b, n):
        """Slots of the next n tokens of sequence b, in order: int64 [n, 2] of (page, slot)."""
        if n < 0:
            raise ValueError("reserve: n must be >= 0")
        P = self.page_tokens
        fr = self.frags[b]
        room = int(P - fr[-1, 1] - fr[-1, 2]) if len(fr) else 0
        take = min(n, room)
        rest = n - take
        k = -(-rest // P)
        if k > len(self.free):
            raise RuntimeError(f"PageTable: {k} pages needed, {len(self.free)} free")
        parts = []
        if take:
            page, end = int(fr[-1, 0]), int(fr[-1, 1] + fr[-1, 2])
            parts.append(np.stack([np.full(take, page), np.arange(end, end + take)], axis=1))
            fr = fr.copy()
            fr[-1, 2] += take
        if k:
            pages = np.array([self.free.pop() for _ in range(k)], dtype=np.int64)
            counts = np.full(k, P, dtype=np.int64)
            counts[-1] = rest - (k - 1) * P
            fr = np.concatenate([fr, np.stack([pages, np.zeros(k, dtype=np.int64), counts], axis=1)])
            idx = np.arange(rest)
            parts.append(np.stack([pages[idx // P], idx % P], axis=1))
        self.frags[b] = fr
        self.version += 1
        return np.concatenate(parts).astype(np.int64) if parts else np.zeros((0, 2), dtype=np.int64)

    def prune(self, b, a, c0, c):
        """Keep tokens [0, a) and [c0, c0 + c) of sequence b; returns (the kept
        suffix's fragments, the pages freed)."""
        old = self.frags[b]
        n = self.length(b)
        if not (0 <= a <= c0 and c >= 0 and c0 + c <= n):
            raise ValueError(f"prune: split (a={a}, c0={c0}, c={c}) outside a sequence of {n} tokens")
        suffix = _cut(old, c0, c0 + c)
        head = _cut(old, 0, a)
        if len(head) and len(suffix) and head[-1, 0] == suffix[0, 0] and head[-1, 1] + head[-1, 2] == suffix[0, 1]:
            # Adjacent pieces of one page merge back (a == c0 leaves the list as it was).
            joint = head[-1:].copy()
            joint[0, 2] += suffix[0, 2]
            new = np.concatenate([head[:-1], joint, suffix[1:]])
        else:
            new = np.concatenate([head, suffix])
        freed = sorted(set(old[:, 0].tolist()) - set(new[:, 0].tolist()))
        self.frags[b] = new
        self.free += freed[::-1]
        self.version += 1
        return suffix, freed

    def release(self, b):
        """Drop sequence b entirely (its pages return to the free list)."""
        self.free += sorted(set(self.frags[b][:, 0].tolist()), reverse=True)
        self.frags[b] = _EMPTY.copy()
        self.version += 1

    def token_slots(self, b):
        """(page, slot) of every token of sequence b in logical order, int64 [n, 2]."""
        fr = self.frags[b]
        if len(fr) == 0:
            return np.zeros((0, 2), dtype=np.int64)
        rep = np.repeat(np.arange(len(fr)), fr[:, 2])
        i = np.arange(len(rep)) - np.repeat(np.cumsum(fr[:, 2]) - fr[:, 2], fr[:, 2])
        return np.stack([fr[rep, 0], fr[rep, 1] + i], axis=1)

    def tile_table(self):
        """int32 [B, max_tiles, 4] and tiles int32 [B] (numpy)."""
        per = [tiles_of(f) for f in self.frags]
        mt = max(1, max(len(t) for t in per))
        tab = np.zeros((self.batch, mt, 4), dtype=np.int32)
        cnt = np.zeros(self.batch, dtype=np.int32)
        for b, ts in enumerate(per):
            tab[b, :len(ts), :3] = ts
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
        for t in list(ks) + list(vs):
            if t.shape[-2] != n or t.numel() != self.kv_heads * n * HEAD_DIM:
                raise ValueError(f"append: every layer's K and V must be [{self.kv_heads}, {n}, {HEAD_DIM}]")
        slots = self.table.reserve(b, n)
        if n == 0:
            return
        idx = torch.from_numpy(slots).to(self.device)
        pages, sl = idx[:, 0], idx[:, 1]
        for kp, vp, k, v in zip(self.k_pools, self.v_pools, ks, vs):
            k = k.reshape(self.kv_heads, n, HEAD_DIM)
            v = v.reshape(self.kv_heads, n, HEAD_DIM)
            kp[pages, :, sl] = k.transpose(0, 1).to(self.dtype)
            vp[pages, :, sl] = v.transpose(0, 1).to(self.dtype)

    def gather(self, layer, b=0):
        """Sequence b's K and V of one layer in logical order, [Hkv, n, D] copies."""
        slots = self.table.token_slots(b)
        if len(slots) == 0:
            z = torch.empty(self.kv_heads, 0, HEAD_DIM, dtype=self.dtype, device=self.device)
            return z, z.clone()
        idx = torch.from_numpy(slots).to(self.device)
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

    def _step_pending(self):
        """True between reserve_step() and the last layer's decode_append of that step:
        the tile table then includes slots no layer has written yet."""
        step = getattr(self, "_step", None)
        return step is not None and step[0] == self.table.version and bool(step[1])

    def _refuse_during_step(self, what):
        if self._step_pending():
            raise RuntimeError(f"PagedKV.{what}: a reserved decode step is incomplete; run decode_append for "
                               "every layer (or cancel_step()) first")

    def cancel_step(self):
        """Drop the slots of an incomplete reserved step (each sequence's last token)."""
        if not self._step_pending():
            return
        for b in range(self.table.batch):
            n = self.table.length(b)
            self.table.prune(b, n - 1, n, 0)
        self._step = None

    def decode(self, layer, q, scale, out=None, split=None):
        """softmax(q·Kᵀ·scale)·V over each sequence's keys of one layer.

        q [B, Hkv, G, D] (G query heads per KV head, last dim contiguous) in the
        pools' dtype; returns out [B, Hkv, G, D]. Enqueued on the current stream.
        """
        self._refuse_during_step("decode")
        _lib.require_gpu(q, what="PagedKV.decode")
        b, hkv, g, d = q.shape
        if b != self.table.batch or hkv != self.kv_heads or d != HEAD_DIM or q.dtype != self.dtype:
            raise ValueError(f"PagedKV.decode: q {tuple(q.shape)} {q.dtype} does not fit the cache")
        if q.stride(3) != 1:
            raise ValueError("PagedKV.decode: q must have a contiguous last dimension")
        if q.device != self.device:
            raise ValueError(f"PagedKV.decode: q is on {q.device}, the pools on {self.device}")
        if not 0 <= layer < self.layers:
            raise IndexError(f"PagedKV.decode: layer {layer} outside [0, {self.layers})")
        if out is None:
            out = torch.empty_like(q)
        elif out.shape != q.shape or out.dtype != q.dtype or out.device != q.device or out.stride(3) != 1:
            raise ValueError("PagedKV.decode: out must match q in shape, dtype and device")
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

    def reserve_step(self):
        """Reserve one slot per sequence for the next decode token (once per step,
        before layer 0); every layer's `decode_append` of that step then writes
        its new K/V row there."""
        self._refuse_during_step("reserve_step")
        for b in range(self.table.batch):
            self.table.reserve(b, 1)
        self._step = (self.table.version, set(range(self.layers)))

    def write_step(self, layer, k_new, v_new):
        """The unfused order of a decode step: write one layer's new K/V rows ([B, Hkv, D] or
        [B, Hkv, 1, D]) into the slots reserve_step() took, with two torch row copies. After
        every layer is written (here or by decode_append), decode() reads the new token."""
        step = getattr(self, "_step", None)
        if step is None or step[0] != self.table.version or layer not in step[1]:
            raise RuntimeError(f"PagedKV.write_step: layer {layer} has no reserved slot in this step")
        b = self.table.batch
        kn = k_new.reshape(b, self.kv_heads, HEAD_DIM)
        vn = v_new.reshape(b, self.kv_heads, HEAD_DIM)
        for i in range(b):
            page, slot = (int(x) for x in self.table.token_slots(i)[-1])
            self.k_pools[layer][page, :, slot] = kn[i]
            self.v_pools[layer][page, :, slot] = vn[i]
        step[1].discard(layer)

    def decode_append(self, layer, q, k_new, v_new, scale, out=None, split=None):
        """One decode step of one layer with the append fused in: k_new/v_new
        [B, Hkv, D] (or [B, Hkv, 1, D]) go to the slots `reserve_step` took, and q
        attends every key of its sequence including the new one. Returns out
        [B, Hkv, G, D]."""
        _lib.require_gpu(q, k_new, v_new, what="PagedKV.decode_append")
        b, hkv, g, d = q.shape
        if b != self.table.batch or hkv != self.kv_heads or d != HEAD_DIM or q.dtype != self.dtype:
            raise ValueError(f"PagedKV.decode_append: q {tuple(q.shape)} {q.dtype} does not fit the cache")
        if not 0 <= layer < self.layers:
            raise IndexError(f"PagedKV.decode_append: layer {layer} outside [0, {self.layers})")
        kn = k_new.reshape(b, hkv, HEAD_DIM) if k_new.dim() == 4 else k_new
        vn = v_new.reshape(b, hkv, HEAD_DIM) if v_new.dim() == 4 else v_new
        for name, t in (("q", q), ("k_new", kn), ("v_new", vn)):
            if t.stride(-1) != 1 or t.dtype != self.dtype or t.device != self.device:
                raise ValueError(f"PagedKV.decode_append: {name} must be {self.dtype} on {self.device}, "
                                 "last dim contiguous")
        if kn.shape != (b, hkv, HEAD_DIM) or vn.shape != (b, hkv, HEAD_DIM):
            raise ValueError("PagedKV.decode_append: k_new/v_new must be [B, Hkv, D]")
        step = getattr(self, "_step", None)
        if step is None or step[0] != self.table.version or layer not in step[1]:
            raise RuntimeError(f"PagedKV.decode_append: layer {layer} has no reserved slot in this step "
                               "(call reserve_step() once per step, then each layer once)")
        if out is None:
            out = torch.empty_like(q)
        elif out.shape != q.shape or out.dtype != q.dtype or out.device != q.device or out.stride(3) != 1:
            raise ValueError("PagedKV.decode_append: out must match q in shape, dtype and device")
        tab, cnt, mt = self.device_table()
        lib = _lib.load()
        kp, vp = self.k_pools[layer], self.v_pools[layer]
        with torch.cuda.device(q.device):
            s = num_splits(b, hkv, TILE * mt, split, ragged=b > 1)
            nbytes = lib.tc_decode_workspace_bytes(b, hkv, g, d, s)
            ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=q.device)
            rc = lib.tc_decode_paged_append_attention(
                q.data_ptr(), _lib.i64x3(*q.stride()[:3]), kp.data_ptr(), vp.data_ptr(), self._strides(),
                kp.shape[0], kp.shape[2], tab.data_ptr(), cnt.data_ptr(), mt,
                kn.data_ptr(), _lib.i64x2(kn.stride(0), kn.stride(1)), vn.data_ptr(),
                _lib.i64x2(vn.stride(0), vn.stride(1)), b, hkv, g, d, _lib.dtype_code(self.dtype), float(scale),
                int(split or 0), ws.data_ptr(), ws.numel(), out.data_ptr(), _lib.i64x3(*out.stride()[:3]),
                _lib.stream_of(q.device))
            _lib.check(rc, "tc_decode_paged_append_attention")
        step[1].discard(layer)
        return out

    def prune(self, b, s, inv_freq):
        """Keep tokens [0, s.a) and [s.c0, s.c0 + s.c) of sequence b (a threadcut
        Split): the dropped span's pages are freed and the kept suffix's keys are
        re-rotated in place by -(c0 - a) positions in every layer. Returns the
        freed page ids."""
        self._refuse_during_step("prune")
        suffix, freed = self.table.prune(b, s.a, s.c0, s.c)
        gap = s.c0 - s.a
        tiles = tiles_of(suffix)
        if gap and len(tiles):
            t = np.zeros((len(tiles), 4), dtype=np.int32)
            t[:, :3] = tiles
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
