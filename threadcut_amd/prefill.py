"""GQA-native prefill attention on MI355X.

Drop-in for the prefill branch of threadcut/attention.py:43-46, which expands
every KV head g = Hq/Hkv times (``repeat_kv``, attention.py:25-27) and runs
SDPA with the boolean mask or ``is_causal``. ``tc_prefill_attention`` reads
the unexpanded K/V instead: a work-group owns 64 query rows of one KV head
(64/g tokens × its g query heads), stages each 64-key tile of K and V in LDS
once for all of them and runs QKᵀ and PV on the matrix cores with an fp32
online softmax. This module checks tensors and passes pointers, strides and
the current stream.
"""
import weakref

import torch

from . import _lib

HEAD_DIM = 128
GROUPS = (1, 2, 4, 8)


def supports(query, key, attention_mask):
    """True if ``prefill_attention`` takes this call: a GPU call in float16 or
    bfloat16 with head_dim 128, g in (1, 2, 4, 8) and no mask or a boolean mask
    [b|1, 1, q, n]."""
    b, hq, q, d = query.shape
    hkv = key.shape[1]
    if not query.is_cuda or d != HEAD_DIM or hq % hkv or hq // hkv not in GROUPS:
        return False
    if query.dtype not in _lib.DTYPES or key.dtype != query.dtype:
        return False
    if attention_mask is None:
        return True
    m = attention_mask
    return (m.dtype == torch.bool and m.dim() == 4 and m.shape[0] in (1, b) and m.shape[1] == 1
            and tuple(m.shape[2:]) == (q, key.shape[2]) and m.device == query.device)


def _strides(t, dims, token_dim=None):
    """Element strides of `dims`; size-1 dims get stride 0 (never stepped), except
    a size-1 token dim of K/V, which gets the row length."""
    st = [t.stride(i) if t.shape[i] > 1 else 0 for i in dims]
    if token_dim is not None and t.shape[token_dim] <= 1:
        st[dims.index(token_dim)] = t.shape[-1]
    return _lib.i64x3(*st)


def _mask_strides(m):
    """Strides of a [mb, q, n] mask view; keys are contiguous (stride 1)."""
    st = _strides(m, (0, 1, 2))
    st[2] = 1
    return st


def num_splits(batch, q_len, n_tokens, q_heads, kv_heads):
    """Key splits a call of this size uses (1 when the query blocks fill the GPU)."""
    s = _lib.load().tc_prefill_num_splits(int(batch), int(q_len), int(n_tokens), int(q_heads), int(kv_heads))
    if s < 0:
        _lib.check(-s, "tc_prefill_num_splits")
    return s


def prefill_attention(query, key, value, attention_mask=None, scale=None, is_causal=False, out=None, splits=None):
    """SDPA(query, repeat_kv(key, g), repeat_kv(value, g), attention_mask, scale,
    is_causal).transpose(1, 2) without expanding K/V.

    query [b, hq, q, d], key/value [b, hkv, n, d] (any strides, contiguous last
    dim), attention_mask None or bool [b|1, 1, q, n] (True = attend).
    ``is_causal`` needs no mask and aligns the queries to the end of the keys
    (identical to SDPA's when q == n). Returns out [b, q, hq, d] (a new
    contiguous tensor unless `out` is given). Rows with no visible key are 0.
    ``splits`` fixes the number of key splits (default: ``num_splits``); more
    than one adds a workspace of fp32 partials and a combine pass.
    """
    _lib.require_gpu(query, key, value, what="prefill_attention")
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        raise ValueError("prefill_attention: expected query [b,hq,q,d], key/value [b,hkv,n,d]")
    if not (query.dtype == key.dtype == value.dtype):
        raise TypeError(f"prefill_attention: dtypes differ ({query.dtype}, {key.dtype}, {value.dtype})")
    b, hq, q, d = query.shape
    hkv, n = key.shape[1], key.shape[2]
    if key.shape != value.shape or key.shape[0] != b or key.shape[3] != d:
        raise ValueError(f"prefill_attention: shapes query {tuple(query.shape)}, key {tuple(key.shape)}, "
                         f"value {tuple(value.shape)} disagree")
    for name, t in (("query", query), ("key", key), ("value", value)):
        if t.stride(3) != 1:
            raise ValueError(f"prefill_attention: {name} must have a contiguous last dimension")
    if attention_mask is not None and is_causal:
        raise ValueError("prefill_attention: pass either attention_mask or is_causal")
    if out is None:
        out = torch.empty((b, q, hq, d), dtype=query.dtype, device=query.device)
    elif out.shape != (b, q, hq, d) or out.dtype != query.dtype or out.device != query.device or out.stride(3) != 1:
        raise ValueError("prefill_attention: out must be [b, q, hq, d] in query's dtype and device")
    mask_ptr, mask_strides, tiles = None, None, None
    if attention_mask is not None:
        m = attention_mask
        if m.dtype != torch.bool or m.dim() != 4 or m.shape[1] != 1 or m.shape[0] not in (1, b) \
                or tuple(m.shape[2:]) != (q, n) or m.device != query.device:
            raise ValueError(f"prefill_attention: attention_mask must be bool [b|1, 1, {q}, {n}] on the device")
        if m.stride(3) != 1 and n > 1:  # the kernels read mask rows as contiguous bytes
            m = m.contiguous()
        tiles = mask_tiles(m, hq, hkv)
        m = m[:, 0]
        mask_ptr, mask_strides = m.data_ptr(), _mask_strides(m)
    scale = scale if scale is not None else d ** -0.5
    lib = _lib.load()
    # The library plans splits for the current device (its CU count).
    with torch.cuda.device(query.device):
        s = int(splits) if splits else num_splits(b, q, n, hq, hkv)
        ws_bytes = lib.tc_prefill_workspace_bytes(b, q, hq, s)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=query.device) if ws_bytes else None
        rc = lib.tc_prefill_attention(
            query.data_ptr(), _strides(query, (0, 1, 2)), key.data_ptr(), _strides(key, (0, 1, 2), 2),
            value.data_ptr(), _strides(value, (0, 1, 2), 2), mask_ptr, mask_strides,
            None if tiles is None else tiles.data_ptr(), 0 if tiles is None else tiles.numel(),
            int(bool(is_causal)), q, n, b, hq, hkv, d, _lib.dtype_code(query.dtype), float(scale), s,
            None if ws is None else ws.data_ptr(), ws_bytes, out.data_ptr(), _strides(out, (0, 1, 2)),
            _lib.stream_of(query.device))
    _lib.check(rc, "tc_prefill_attention")
    return out


# The tile map of the last mask seen. transformers builds one mask per forward
# pass and hands the same tensor to every layer, so the map is built once per
# pass; it is rebuilt when the mask object, its version or the geometry change.
_tile_cache = None


def mask_tiles(mask, q_heads, kv_heads):
    """uint8 tile map of a bool mask [b|1, 1, q, n] (``tc_prefill_mask_tiles``), cached per mask."""
    global _tile_cache
    key = (mask._version, tuple(mask.shape), tuple(mask.stride()), mask.data_ptr(), q_heads, kv_heads)
    c = _tile_cache
    if c is not None and c[0]() is mask and c[1] == key:
        return c[2]
    m = mask[:, 0]
    mb = m.shape[0] if m.shape[0] > 1 and m.stride(0) != 0 else 1
    q, n = m.shape[1], m.shape[2]
    lib = _lib.load()
    nbytes = lib.tc_prefill_tiles_bytes(q, n, mb, q_heads, kv_heads)
    tiles = torch.empty(max(1, nbytes), dtype=torch.uint8, device=mask.device)
    st = _mask_strides(m)
    if mb == 1:
        st[0] = 0
    with torch.cuda.device(mask.device):
        rc = lib.tc_prefill_mask_tiles(m.data_ptr(), st, mb, q, n, q_heads, kv_heads, tiles.data_ptr(),
                                       tiles.numel(), _lib.stream_of(mask.device))
    _lib.check(rc, "tc_prefill_mask_tiles")
    _tile_cache = (weakref.ref(mask), key, tiles)
    return tiles
