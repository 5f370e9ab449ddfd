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
  slots, entries ``{page, first slot, rows, first logical position}``
  (``tc_decode_paged_attention``). Attention over a set of keys does not
  depend on their order, so holes left by prunes cost nothing.
- The prune's only device work is ``tc_paged_rotate_keys``: C's keys rotated
  in place by -(c0 - a) positions with the reference's rotation
  (threadcut/kv.py:20-25), for every layer in one launch. V is not touched.

``PageTable`` is the bookkeeping alone (no device; its fragment arithmetic is the
host code of ``tc_page_tiles``, ``tc_page_prune`` and ``tc_page_token_offsets``),
``PagedKV`` adds the pools.
"""
import ctypes
import weakref

import numpy as np
import torch
import torch.nn.functional as F
from transformers import DynamicCache
from transformers.cache_utils import DynamicLayer

from . import _lib
from .flash_decode import HEAD_DIM, _on_device, _plan
from .kv import rope_table
from .prefill import GROUPS

TILE = 16  # rows per tile-table entry (the decode kernel's tile)
_I64P = ctypes.POINTER(ctypes.c_int64)


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


def _to_device(arr, device):
    """A host numpy array as a device tensor: staged in pinned memory and copied on the
    current stream without a host wait (torch keeps the staging block until the copy ran)."""
    return torch.from_numpy(np.ascontiguousarray(arr)).pin_memory().to(device, non_blocking=True)


def _addr(a):
    return a.__array_interface__["data"][0]


def _frag_arg(frags):
    f = frags
    if not (isinstance(f, np.ndarray) and f.dtype == np.int64 and f.ndim == 2 and f.flags.c_contiguous):
        f = np.ascontiguousarray(np.asarray(frags, dtype=np.int64).reshape(-1, 3))
    return f, _addr(f), len(f)


def _tiles(frags, page_tokens, first_pos=0):
    """Tile entries {page, first slot, rows, logical start} of a fragment array of pages of
    page_tokens slots, int32 [T, 4] (tc_page_tiles): each fragment cut at multiples of 16
    slots."""
    lib = _lib.load()
    f, fp, nf = _frag_arg(frags)
    n = lib.tc_page_tiles(fp, nf, int(page_tokens), int(first_pos), None, 0)
    if n < 0:
        _lib.check(-n, "tc_page_tiles")
    out = np.empty((n, 4), dtype=np.int32)
    if n:
        _lib.check(0 if lib.tc_page_tiles(fp, nf, int(page_tokens), int(first_pos), _addr(out), n) == n
                   else _lib.TC_ERR_INVALID_ARGUMENT, "tc_page_tiles")
    return out


def tiles_of(frags, page_tokens):
    """Tile entries (page, first slot, rows) of a fragment array of pages of page_tokens
    slots, int32 [T, 3]: each fragment is cut at multiples of 16 slots, so full tiles are
    16-slot aligned."""
    return np.ascontiguousarray(_tiles(frags, page_tokens)[:, :3])


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
        suffix's fragments, the pages freed) (tc_page_prune)."""
        old = self.frags[b]
        n = self.length(b)
        if not (0 <= a <= c0 and c >= 0 and c0 + c <= n):
            raise ValueError(f"prune: split (a={a}, c0={c0}, c={c}) outside a sequence of {n} tokens")
        f, fp, nf = _frag_arg(old)
        # One buffer: kept (nf + 1 rows), suffix (nf rows), freed (nf), counts (3).
        buf = np.empty(7 * nf + 6, dtype=np.int64)
        base = _addr(buf)
        rc = _lib.load().tc_page_prune(fp, nf, self.page_tokens, int(a), int(c0), int(c), base,
                                       base + 8 * (3 * nf + 3), base + 8 * (6 * nf + 3),
                                       ctypes.cast(base + 8 * (7 * nf + 3), _I64P))
        _lib.check(rc, "tc_page_prune")
        nk, ns, nfr = (int(x) for x in buf[7 * nf + 3:])
        self.frags[b] = buf[:3 * nk].reshape(nk, 3).copy()
        freed = buf[6 * nf + 3:6 * nf + 3 + nfr].tolist()
        self.free += freed[::-1]
        self.version += 1
        return buf[3 * nf + 3:3 * nf + 3 + 3 * ns].reshape(ns, 3).copy(), freed

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
        """int32 [B, max_tiles, 4] and tiles int32 [B] (numpy): entries {page, first slot,
        rows, first logical position} in logical order."""
        per = [_tiles(f, self.page_tokens) for f in self.frags]
        mt = max(1, max(len(t) for t in per))
        tab = np.zeros((self.batch, mt, 4), dtype=np.int32)
        cnt = np.zeros(self.batch, dtype=np.int32)
        for b, ts in enumerate(per):
            tab[b, :len(ts)] = ts
            cnt[b] = len(ts)
        return tab, cnt

    def token_offsets(self, page_bytes, slot_bytes, pitch=None):
        """int32 [B, pitch]: byte offset of every logical token's row within a head slab of
        the pools (page * page_bytes + slot * slot_bytes); past a sequence's end, INT32_MIN,
        which no buffer range covers."""
        n = max([self.length(b) for b in range(self.batch)] + [1])
        pitch = max(n, int(pitch or 0))
        off = np.empty((self.batch, pitch), dtype=np.int32)
        lib = _lib.load()
        for b in range(self.batch):
            f, fp, nf = _frag_arg(self.frags[b])
            if lib.tc_page_token_offsets(fp, nf, self.page_tokens, int(page_bytes), int(slot_bytes), _addr(off[b]),
                                         pitch) < 0:
                raise RuntimeError("PageTable.token_offsets: pools of 2 GiB or more need 64-bit offsets")
        return off


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
        # The pools' own device, with its index ("cuda" alone names the current device).
        self.device = self.k_pools[0].device if self.k_pools else torch.device(
            "cuda", torch.cuda.current_device() if dev.index is None else dev.index)
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
        idx = _to_device(slots, self.device)
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
        idx = _to_device(slots, self.device)
        k = self.k_pools[layer][idx[:, 0], :, idx[:, 1]].transpose(0, 1).contiguous()
        v = self.v_pools[layer][idx[:, 0], :, idx[:, 1]].transpose(0, 1).contiguous()
        return k, v

    def device_table(self):
        """(tile table int32 [B, max_tiles, 4], tiles int32 [B], max_tiles) on the device."""
        ver = self.table.version
        if self._dev_table is None or self._dev_table[0] != ver:
            tab, cnt = self.table.tile_table()
            self._dev_table = (ver, _to_device(tab, self.device), _to_device(cnt, self.device),
                               tab.shape[1])
        return self._dev_table[1:]

    def device_offsets(self):
        """(token offsets int32 [B, pitch], pitch) on the device: the byte offset of each logical
        token's row in a head slab of the pools (PageTable.token_offsets), for the paged prefill
        and the device-length decode step."""
        ver = self.table.version
        if getattr(self, "_dev_off", None) is None or self._dev_off[0] != ver:
            st = self.k_pools[0].stride()
            off = self.table.token_offsets(st[0] * 2, st[2] * 2)
            self._dev_off = (ver, _to_device(off, self.device), off.shape[1])
        return self._dev_off[1:]

    def prefill(self, layer, query, scale, mask=None, causal=False, out=None):
        """The prefill branch of threadcut/attention.py:43-46 over the pools: query
        [B, Hq, q, D] (any strides, last dim contiguous) attends the first n keys of every
        sequence (n = the sequences' common length; the last q of them are the queries'
        own tokens), in logical order, with no mask, is_causal, or a boolean mask
        [B|1, 1, q, n]. Returns [B, q, Hq, D] (the reference's transposed output)."""
        from . import prefill as pf

        self._refuse_during_step("prefill", layer)
        _lib.require_gpu(query, what="PagedKV.prefill")
        b, hq, ql, d = query.shape
        lens = {self.table.length(i) for i in range(self.table.batch)}
        if b != self.table.batch or d != HEAD_DIM or query.dtype != self.dtype or query.device != self.device:
            raise ValueError(f"PagedKV.prefill: query {tuple(query.shape)} {query.dtype} does not fit the cache")
        if len(lens) != 1:
            raise ValueError(f"PagedKV.prefill: sequences of different lengths {sorted(lens)}")
        n = lens.pop()
        if not 0 <= ql <= n or hq % self.kv_heads:
            raise ValueError(f"PagedKV.prefill: {ql} queries over {n} keys, {hq} query heads")
        if out is None:
            out = torch.empty((b, ql, hq, d), dtype=query.dtype, device=query.device)
        if ql == 0:
            return out
        if mask is not None and causal:
            raise ValueError("PagedKV.prefill: pass either a mask or causal")
        off, pitch = self.device_offsets()
        tiles, tiles_bytes, mptr, mst = None, 0, None, _lib.i64x3(0, 0, 1)
        if mask is not None:
            m = mask
            if m.dtype != torch.bool or m.dim() != 4 or m.shape[1] != 1 or m.shape[0] not in (1, b) \
                    or tuple(m.shape[2:]) != (ql, n) or m.device != self.device:
                raise ValueError(f"PagedKV.prefill: the mask must be bool [B|1, 1, {ql}, {n}] on the pools' device")
            if m.stride(3) != 1 and n > 1:  # the kernel reads mask rows as contiguous bytes
                m = m.contiguous()
            tiles = pf.mask_tiles(m, hq, self.kv_heads)
            tiles_bytes = tiles.numel()
            m = m[:, 0]
            mptr, mst = m.data_ptr(), pf._mask_strides(m)
        lib = _lib.load()
        kp, vp = self.k_pools[layer], self.v_pools[layer]
        with torch.cuda.device(self.device):
            splits = pf.num_splits(b, ql, n, hq, self.kv_heads)
            nbytes = lib.tc_prefill_workspace_bytes(b, ql, hq, splits)
            ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=self.device)
            rc = lib.tc_prefill_paged_attention(
                query.data_ptr(), pf._strides(query, (0, 1, 2)), kp.data_ptr(), vp.data_ptr(), self._strides(),
                kp.shape[0], off.data_ptr(), pitch, mptr, mst,
                None if tiles is None else tiles.data_ptr(), tiles_bytes, int(bool(causal)), ql, n, b, hq,
                self.kv_heads, d, _lib.dtype_code(self.dtype), float(scale), splits, ws.data_ptr(), ws.numel(),
                out.data_ptr(), pf._strides(out, (0, 1, 2)), _lib.stream_of(self.device))
            _lib.check(rc, "tc_prefill_paged_attention")
        return out

    def _step_pending(self, layer=None):
        """True between reserve_step() and the last layer's decode_append of that step:
        the tile table then includes slots not every layer has written yet. With `layer`,
        True only while that layer's own row of the step is unwritten."""
        step = getattr(self, "_step", None)
        if step is None or step[0] != self.table.version:
            return False
        return bool(step[1]) if layer is None else layer in step[1]

    def _refuse_during_step(self, what, layer=None):
        """Refuse a read of the tile table while the reserved step's slots are unwritten: in
        every layer (layer None: prune, a new reservation), or in the layer to be read."""
        if self._step_pending(layer):
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
        self._refuse_during_step("decode", layer)
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
        _, nbytes = _plan(q.device.index, b, hkv, g, d, TILE * mt, split, b > 1)
        with _on_device(q.device):
            ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
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
        [B, Hkv, 1, D]) into the slots reserve_step() took, with two torch row copies. Once a
        layer's row is written (here or by decode_append), decode() and prefill() of that layer
        read the new token; prune() and the next reserve_step() wait for every layer."""
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
        _, nbytes = _plan(q.device.index, b, hkv, g, d, TILE * mt, split, b > 1)
        with _on_device(q.device):
            ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
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

    def decode_append_at(self, layer, q, k_new, v_new, lens, scale, out=None):
        """decode_append with the sequence lengths on the device (int32 [B], tokens before the
        step), for a captured step: the new rows go to logical positions lens[b], whose slots
        must already be in the table (reserved ahead), and q attends positions [0, lens[b]].
        Nothing here reads lens on the host, so a graph of this call stays valid while lens
        advances; the table must not change meanwhile."""
        b, hkv, g, d = q.shape
        kn = k_new.reshape(b, hkv, HEAD_DIM)
        vn = v_new.reshape(b, hkv, HEAD_DIM)
        for name, t in (("q", q), ("k_new", kn), ("v_new", vn)):
            if t.stride(-1) != 1 or t.dtype != self.dtype or t.device != self.device:
                raise ValueError(f"PagedKV.decode_append_at: {name} must be {self.dtype} on {self.device}, "
                                 "last dim contiguous")
        if lens.dtype != torch.int32 or lens.shape != (b,) or lens.device != self.device:
            raise ValueError("PagedKV.decode_append_at: lens must be int32 [B] on the pools' device")
        if out is None:
            out = torch.empty_like(q)
        tab, cnt, mt = self.device_table()
        off, pitch = self.device_offsets()
        lib = _lib.load()
        kp, vp = self.k_pools[layer], self.v_pools[layer]
        _, nbytes = _plan(self.device.index, b, hkv, g, d, TILE * mt, None, b > 1)
        with _on_device(self.device):
            ws = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
            rc = lib.tc_decode_paged_append_attention_at(
                q.data_ptr(), _lib.i64x3(*q.stride()[:3]), kp.data_ptr(), vp.data_ptr(), self._strides(),
                kp.shape[0], kp.shape[2], tab.data_ptr(), cnt.data_ptr(), mt, off.data_ptr(), pitch, lens.data_ptr(),
                kn.data_ptr(), _lib.i64x2(kn.stride(0), kn.stride(1)), vn.data_ptr(),
                _lib.i64x2(vn.stride(0), vn.stride(1)), b, hkv, g, d, _lib.dtype_code(self.dtype), float(scale), 0,
                ws.data_ptr(), ws.numel(), out.data_ptr(), _lib.i64x3(*out.stride()[:3]), _lib.stream_of(self.device))
            _lib.check(rc, "tc_decode_paged_append_attention_at")
        return out

    def prune(self, b, s, inv_freq):
        """Keep tokens [0, s.a) and [s.c0, s.c0 + s.c) of sequence b (a threadcut
        Split): the dropped span's pages are freed and the kept suffix's keys are
        re-rotated in place by -(c0 - a) positions in every layer. Returns the
        freed page ids."""
        self._refuse_during_step("prune")
        suffix, freed = self.table.prune(b, s.a, s.c0, s.c)
        gap = s.c0 - s.a
        tiles = tiles_of(suffix, self.table.page_tokens)
        if gap and len(tiles):
            t = np.zeros((len(tiles), 4), dtype=np.int32)
            t[:, :3] = tiles
            td = _to_device(t, self.device)
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


# ---------------------------------------------------------------------------
# The paged cache behind transformers' cache interface.
# ---------------------------------------------------------------------------

# PagedLayers by the address of their K pool: update() returns the pools, and
# the "threadcut" attention finds the layer behind them here. The entries are
# weak: a cache that nothing else holds is freed with its pools, and its
# entries leave the registry with it.
_LAYERS = weakref.WeakValueDictionary()


def layer_of(key):
    """The PagedLayer whose K pool `key` is, or None."""
    if not isinstance(key, torch.Tensor) or not key.is_cuda:
        return None
    layer = _LAYERS.get(key.data_ptr())
    if layer is None or layer.owner.kv is None or layer.owner.kv.k_pools[layer.index] is not key:
        return None
    return layer


class PagedCacheState:
    """What the layers of one paged cache share: the PagedKV (made at the first update,
    when the head count, dtype and device are known), the fused-append switch and, while
    a DecodeGraph holds the cache, the device lengths of its captured step."""

    def __init__(self, num_layers, num_pages, page_tokens, batch, fused_append):
        self.num_layers, self.num_pages, self.page_tokens, self.batch = num_layers, num_pages, page_tokens, batch
        self.fused_append = fused_append
        self.kv = None
        self.layers = []
        self.device_lens = None
        self.in_graph_step = False
        self._slots = {}

    def ensure_pools(self, like):
        if self.kv is None:
            if like.dim() != 4 or like.shape[0] != self.batch or like.shape[-1] != HEAD_DIM:
                raise ValueError(f"paged cache: K/V {tuple(like.shape)} for a batch of {self.batch} at head_dim "
                                 f"{HEAD_DIM}")
            self.kv = PagedKV(self.num_layers, like.shape[1], self.num_pages, self.page_tokens, batch=self.batch,
                              dtype=like.dtype, device=like.device)

    def check_not_captured(self, what):
        if self.device_lens is not None and not self.in_graph_step:
            raise RuntimeError(f"paged cache {what}: a DecodeGraph holds this cache; close() it first")

    def write(self, layer, keys, values):
        """Rows of positions [layer.n, layer.n + add) of every sequence into the layer's pools,
        reserving the slots when this is the first layer to reach them."""
        kv = self.kv
        add = keys.shape[-2]
        need = layer.n + add - kv.table.length(0)
        if need > 0:
            for b in range(self.batch):
                kv.table.reserve(b, need)
        kp, vp = kv.k_pools[layer.index], kv.v_pools[layer.index]
        for b in range(self.batch):
            sl = self.slots_on_device(b, layer.n, layer.n + add)
            kp[sl[:, 0], :, sl[:, 1]] = keys[b].transpose(0, 1).to(kv.dtype)
            vp[sl[:, 0], :, sl[:, 1]] = values[b].transpose(0, 1).to(kv.dtype)

    def slots_on_device(self, b, lo, hi):
        """(page, slot) of sequence b's positions [lo, hi) on the device; every layer of a
        step writes the same positions, so the upload is kept for the table version."""
        key = (self.kv.table.version, b, lo, hi)
        hit = self._slots.get(key)
        if hit is None:
            if self._slots and next(iter(self._slots))[0] != key[0]:
                self._slots.clear()
            hit = self._slots[key] = _to_device(self.kv.table.token_slots(b)[lo:hi], self.kv.device)
        return hit

    def reserve_step_for(self, layer):
        """A decode step's slot per sequence: reserved by the first layer of the step."""
        if layer.n == self.kv.table.length(0):
            self.kv.reserve_step()


class PagedLayer(DynamicLayer):
    """A transformers cache layer whose K/V rows live in the pools of a PagedKV shared by
    every layer of the cache (one page table for all).

    update() writes the new tokens' rows into their slots and returns the layer's K and V
    pools, which the "threadcut" attention recognises (layer_of) and serves with the paged
    kernels: decode over the tile table, prefill through the token offsets. With
    fused_append a one-token update reserves the step's slot and leaves the row pending;
    the decode kernel writes it while it attends.
    """

    def __init__(self, owner, index):
        super().__init__()
        self.owner, self.index = owner, index
        self.n = 0
        self.pending = None

    @property
    def kv(self):
        return self.owner.kv

    def lazy_initialization(self, key_states, value_states):
        super().lazy_initialization(key_states, value_states)
        self.owner.ensure_pools(key_states)
        self.n = 0

    def flush(self):
        """Write a pending row that no attention call consumed. In a captured step (device
        lengths) only the decode kernel can place the row, at lens[b]; a row left pending
        there would be lost, so that raises."""
        if self.pending is not None:
            k, v = self.pending
            self.pending = None
            if self.owner.device_lens is not None:
                raise RuntimeError(
                    "paged cache: a one-token update of a captured decode step reached no decode attention "
                    "call (an attention mask, or a second update before attention); its K/V row would be lost")
            self.kv.write_step(self.index, k, v)

    def update(self, key_states, value_states, *args, **kwargs):
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        self.owner.check_not_captured("update")
        self.flush()
        add = key_states.shape[-2]
        if add == 1 and self.owner.device_lens is not None:
            self.pending = (key_states, value_states)  # written at lens[b] by the captured kernel
        elif add == 1 and self.owner.fused_append and key_states.is_cuda:
            self.owner.reserve_step_for(self)
            self.pending = (key_states, value_states)
        else:
            self.owner.write(self, key_states, value_states)
        self.n += add
        kp = self.kv.k_pools[self.index]
        _LAYERS[kp.data_ptr()] = self
        return kp, self.kv.v_pools[self.index]

    def get_seq_length(self):
        return self.n if self.is_initialized else 0

    def crop(self, max_length):
        raise NotImplementedError("PagedLayer.crop: shorten a paged cache with kv.splice (a prune) instead")


def new_paged_cache(config, num_pages, page_tokens=64, batch=1, fused_append=True):
    """A DynamicCache whose layers keep their K/V in page pools (PagedKV): the engine's
    cache (threadcut/kv.py:95-98) in the layout the reference's README.md:141-144 proposes.
    Use it with the "threadcut" attention; kv.splice prunes it (pages of the dropped span
    freed, the kept suffix's keys re-rotated in place)."""
    cache = DynamicCache(config=config)
    state = PagedCacheState(len(cache.layers), num_pages, page_tokens, batch, fused_append)
    cache.layers = [PagedLayer(state, i) for i in range(len(cache.layers))]
    state.layers = cache.layers
    return cache


def state_of(cache):
    """The PagedCacheState of a new_paged_cache() cache, or None."""
    layers = getattr(cache, "layers", None)
    if layers and all(isinstance(l, PagedLayer) for l in layers):
        return layers[0].owner
    return None


def attention(layer, query, attention_mask, scaling):
    """The "threadcut" attention for a paged layer: query [B, Hq, q, D] -> [B, q, Hq, D]."""
    b, hq, q, d = query.shape
    kv = layer.kv
    hkv = kv.kv_heads
    g = hq // hkv
    if q == 1 and attention_mask is None:
        out = torch.empty((b, 1, hq, d), dtype=query.dtype, device=query.device)
        qg, og = query.reshape(b, hkv, g, d), out.view(b, hkv, g, d)
        if layer.pending is not None:
            k_new, v_new = layer.pending
            layer.pending = None
            if layer.owner.device_lens is not None:
                kv.decode_append_at(layer.index, qg, k_new, v_new, layer.owner.device_lens, scaling, out=og)
            else:
                kv.decode_append(layer.index, qg, k_new, v_new, scaling, out=og)
        else:
            kv.decode(layer.index, qg, scaling, out=og)
        return out
    layer.flush()
    is_causal = attention_mask is None and q > 1 and q == layer.n
    m = attention_mask
    if g in GROUPS and (m is None or (m.dtype == torch.bool and m.dim() == 4 and m.shape[1] == 1)):
        return kv.prefill(layer.index, query, scaling, m, is_causal)
    # Other masks and group sizes: the reference's route (repeat_kv + SDPA) on the gathered keys.
    ks, vs = zip(*[kv.gather(layer.index, i) for i in range(b)])
    k, v = torch.stack(ks), torch.stack(vs)
    out = F.scaled_dot_product_attention(query, k.repeat_interleave(g, 1), v.repeat_interleave(g, 1),
                                         attn_mask=m, scale=scaling, is_causal=is_causal)
    return out.transpose(1, 2).contiguous()
