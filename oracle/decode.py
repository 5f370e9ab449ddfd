"""Oracle of the split-KV GQA decode — TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Functions and the reference lines each restates:

- ``flash_decode_partial``: the Triton ``_partial`` program of
  threadcut/flash_decode.py:21-54, in numpy float32, block by block (the
  BLOCK-token online-softmax update with the m_safe/-inf guards, then
  out = acc / l and lse = m + log l).
- ``flash_decode_combine``: threadcut/flash_decode.py:68-69 (softmax over the
  split axis of lse, weighted sum, cast to the input dtype).
- ``decode_attention``: threadcut/flash_decode.py:57-69 end to end.
- ``folded_sdpa``: the decode branch of threadcut/attention.py:40-42 — torch
  SDPA with the g query heads folded into a length-g query against the
  unexpanded cache. This IS the reference's CPU path (its code for non-CUDA
  tensors); bench.py times it as the CPU baseline.
- ``attention_f64``: closed form softmax(q·kᵀ·scale)·v in float64.
- ``decode_ragged``: per-sequence ``attention_f64`` over k[b, :, :len_b].

Pins (tests/test_oracle_decode.py): ``flash_decode_partial``+``combine``
against the float64 closed form and against torch's own SDPA (a library
routine), brute-force loops on tiny shapes, and invariants a dropped term or
wrong index breaks — split length does not change the result; constant V
gives that row; q = 0 gives mean(V); a single split's combine is the
identity; n = 0 gives zeros (the reference's empty sum); large scales stay
finite. Mutated copies of the oracle (no rescale, no m_safe guard,
transposed operands) are shown to fail those pins.
"""
import numpy as np


def to_dtype_bits(x32, dtype):
    """float32 array -> float16 array, or bfloat16 as uint16 bits (round to nearest even)."""
    x32 = np.asarray(x32, np.float32)
    if dtype == "float16":
        return x32.astype(np.float16)
    if dtype == "bfloat16":
        u = x32.view(np.uint32).astype(np.uint64)
        nan = (u & 0x7FFFFFFF) > 0x7F800000
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        q = ((u >> 16) | 0x40).astype(np.uint16)
        return np.where(nan, q, r)
    raise ValueError(dtype)


def from_dtype_bits(x, dtype):
    """float16 array, or bfloat16 uint16 bits -> float32."""
    if dtype == "float16":
        return np.asarray(x, np.float16).astype(np.float32)
    if dtype == "bfloat16":
        return (np.asarray(x, np.uint16).astype(np.uint32) << 16).view(np.float32)
    raise ValueError(dtype)


def flash_decode_partial(q, k, v, scale, split=256, block=16):
    """threadcut/flash_decode.py:21-54 over grid (hkv, cdiv(n, split)).

    q [hkv, g, d], k/v [hkv, n, d] as float32 arrays (already upcast from the
    storage dtype, as the kernel's loads do). Returns o [S, hkv, g, d] and
    lse [S, hkv, g], float32.
    """
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    hkv, g, d = q.shape
    n = k.shape[1]
    S = -(-n // split)
    scale = np.float32(scale)
    o = np.empty((S, hkv, g, d), np.float32)
    lse = np.empty((S, hkv, g), np.float32)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        for s in range(S):
            m = np.full((hkv, g), -np.inf, np.float32)                     # :31
            l = np.zeros((hkv, g), np.float32)                              # :32
            acc = np.zeros((hkv, g, d), np.float32)                         # :33
            for off in range(s * split, s * split + split, block):         # :35
                idx = off + np.arange(block)
                valid = idx < n                                             # :37
                kb = np.zeros((hkv, block, d), np.float32)                  # :38 other=0
                vb = np.zeros((hkv, block, d), np.float32)                  # :39
                kb[:, valid] = k[:, idx[valid]]
                vb[:, valid] = v[:, idx[valid]]
                qk = np.einsum("hgd,hnd->hgn", q, kb).astype(np.float32) * scale   # :42
                qk = np.where(valid[None, None, :], qk, np.float32(-np.inf))     # :43
                m_new = np.maximum(m, qk.max(axis=2))                       # :44
                m_safe = np.where(m_new == -np.inf, np.float32(0), m_new)   # :45
                p = np.exp(qk - m_safe[:, :, None])                          # :46
                alpha = np.exp(m - m_safe)                                   # :47
                l = l * alpha + p.sum(axis=2)                                # :48
                acc = acc * alpha[:, :, None] + np.einsum("hgn,hnd->hgd", p, vb).astype(np.float32)  # :49
                m = m_new                                                    # :50
            o[s] = acc / np.where(l == 0, np.float32(1), l)[:, :, None]      # :51
            lse[s] = np.where(l == 0, np.float32(-np.inf), m + np.log(l))    # :52
    return o, lse


def flash_decode_combine(o, lse):
    """threadcut/flash_decode.py:68-69 before the cast: sum_s softmax_s(lse) * o_s (float32).

    With no splits (n = 0) the sum is empty and the result is zeros.
    """
    o = np.asarray(o, np.float32)
    lse = np.asarray(lse, np.float32)
    if o.shape[0] == 0:
        return np.zeros(o.shape[1:], np.float32)
    with np.errstate(invalid="ignore"):
        mx = lse.max(axis=0, keepdims=True)
        e = np.exp(lse - mx)
        w = e / e.sum(axis=0, keepdims=True)
    return (o * w[..., None]).sum(axis=0).astype(np.float32)


def decode_attention(q, k, v, scale, split=256, block=16):
    """threadcut/flash_decode.py:57-69 in float32 (the caller casts to the storage dtype)."""
    o, lse = flash_decode_partial(q, k, v, scale, split, block)
    return flash_decode_combine(o, lse)


def attention_f64(q, k, v, scale):
    """softmax(q·kᵀ·scale)·v in float64; q [..., g, d], k/v [..., n, d]. n = 0 gives zeros."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    if k.shape[-2] == 0:
        return np.zeros(q.shape, np.float64)
    s = np.einsum("...gd,...nd->...gn", q, k) * float(scale)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("...gn,...nd->...gd", p, v)


def decode_ragged(q, k, v, lens, scale):
    """Per-sequence closed form: q [B, hkv, g, d], k/v [B, hkv, N, d], lens [B]."""
    out = np.zeros(np.shape(q), np.float64)
    for b, n in enumerate(np.asarray(lens)):
        out[b] = attention_f64(q[b], k[b, :, :int(n)], v[b, :, :int(n)], scale)
    return out


def folded_sdpa(query, key, value, scaling):
    """The reference's CPU decode path, threadcut/attention.py:40-42 (torch tensors).

    query [b, hq, 1, d], key/value [b, hkv, n, d] -> [b, hq, 1, d] in the input dtype.
    """
    import torch.nn.functional as F

    b, hq, _, d = query.shape
    hkv = key.shape[1]
    g = hq // hkv
    return F.scaled_dot_product_attention(query.reshape(b, hkv, g, d), key, value,
                                          scale=scaling).reshape(b, hq, 1, d)
