"""Oracle of the RoPE delta-shift and the suffix splice — TEST INFRASTRUCTURE ONLY.

Functions and the reference lines each restates:

- ``default_inv_freq``: transformers' default RoPE frequencies
  1 / theta^(arange(0, d, 2) / d) in float32 (the ``inv_freq`` the reference
  engine reads, threadcut/engine.py:33; transformers
  models/qwen3/modeling_qwen3.py:121).
- ``rope_table``: threadcut/kv.py:22-23 — angle = delta * inv_freq.float(),
  emb = cat(angle, angle), emb.cos(), emb.sin(), with torch on the CPU exactly
  as the reference evaluates it; returns the lower halves (the upper halves
  repeat them).
- ``shift_keys``: threadcut/kv.py:15-25 — fp32 k*cos(emb) + rotate_half(k)*sin(emb)
  as separately rounded numpy float32 operations, then round to the storage
  dtype.
- ``splice_growing``: threadcut/kv.py:83-92 — K[a:a+c] <- shift(K[c0:c0+c], -gap)
  (a plain copy when gap = 0), V[a:a+c] <- V[c0:c0+c], sources read before
  any write (the reference clones), n = a + c, other rows unchanged.
- ``splice_copy``: threadcut/kv.py:34-41 — index_select of [0, a) ∪ [c0, c0+c),
  then shift of rows [a:] when c and gap.
- ``splice_growing_torch``: threadcut/kv.py:20-25 and :83-92 as the reference
  runs them on host tensors (torch ops, per layer): the CPU path that bench.py
  times as the splice's baseline.

Pins (tests/test_oracle_splice.py): ``rope_table`` against float64 cos/sin;
``shift_keys`` bit for bit against the reference's torch op sequence on the
same data and against the T1 composition identity of the reference's tests
(shift(rope(k, 900), -350) = rope(k, 550), threadcut's tests/test_core.py:67-74,
RoPE from transformers' own rotary embedding); shift(0) = identity, per-pair
norms preserved, shift(d1)∘shift(d2) ≈ shift(d1+d2); ``splice_growing``
against ``splice_copy`` for Split(10,17,20) (overlapping) and
Split(12,12,0) as in tests/test_core.py:104-121, against a per-row brute force,
and with rows outside [a, a+c) checked unchanged; ``splice_growing_torch``
bit for bit against ``splice_growing``.
"""
import numpy as np

from .decode import from_dtype_bits, to_dtype_bits


def default_inv_freq(theta, head_dim):
    """float32 [head_dim/2]: 1 / theta ** (arange(0, d, 2) / d) (transformers' default RoPE)."""
    import torch

    return (1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))).float()


def rope_table(delta, inv_freq):
    """(cos, sin) float32 [d/2] of angle = delta * inv_freq, via threadcut/kv.py:22-23's torch ops."""
    import torch

    f = torch.as_tensor(inv_freq).detach().to("cpu").float()
    angle = delta * f
    emb = torch.cat((angle, angle))
    half = f.numel()
    return emb.cos()[:half].numpy().copy(), emb.sin()[:half].numpy().copy()


def shift_keys(keys, cos, sin, dtype="float16"):
    """threadcut/kv.py:25 on storage-dtype keys [..., d] with a given (cos, sin) table.

    keys: float16 array, or bfloat16 as uint16 bits. Returns the same kind.
    """
    k = from_dtype_bits(keys, dtype)
    half = k.shape[-1] // 2
    c = np.asarray(cos, np.float32)
    s = np.asarray(sin, np.float32)
    k1, k2 = k[..., :half], k[..., half:]
    # k * cos(emb) + rotate_half(k) * sin(emb), every product and sum rounded to fp32.
    lo = (k1 * c).astype(np.float32) + (-k2 * s).astype(np.float32)
    hi = (k2 * c).astype(np.float32) + (k1 * s).astype(np.float32)
    return to_dtype_bits(np.concatenate((lo, hi), axis=-1).astype(np.float32), dtype)


def splice_growing(kbuf, vbuf, n, a, c0, c, cos=None, sin=None, dtype="float16"):
    """threadcut/kv.py:83-92 on copies of [..., cap, d] buffers; returns (kbuf', vbuf', n')."""
    kbuf = np.array(kbuf, copy=True)
    vbuf = np.array(vbuf, copy=True)
    if c:
        k = kbuf[..., c0:c0 + c, :].copy()          # read C before any write (the clone)
        if c0 != a:
            k = shift_keys(k, cos, sin, dtype)
        v = vbuf[..., c0:c0 + c, :].copy()
        kbuf[..., a:a + c, :] = k
        vbuf[..., a:a + c, :] = v
    return kbuf, vbuf, a + c


def splice_copy(keys, values, a, c0, c, cos=None, sin=None, dtype="float16"):
    """threadcut/kv.py:34-41 on [..., n, d] arrays; returns new (keys, values) of a + c tokens."""
    keep = np.concatenate((np.arange(0, a), np.arange(c0, c0 + c)))
    k = np.take(keys, keep, axis=-2)
    v = np.take(values, keep, axis=-2)
    if c and c0 != a:
        k[..., a:, :] = shift_keys(k[..., a:, :], cos, sin, dtype)
    return k, v


def splice_growing_torch(kbufs, vbufs, a, c0, c, inv_freq):
    """threadcut/kv.py:83-92 over every layer, in place, with torch on host tensors.

    kbufs/vbufs: lists of [B, H, cap, D] fp16/bf16 CPU tensors. Per layer, as
    the reference: K[a:a+c] <- shift_keys(K[c0:c0+c], -gap) (kv.py:20-25: fp32
    k*cos(emb) + rotate_half(k)*sin(emb), cast back), V[a:a+c] <- clone of
    V[c0:c0+c].
    """
    import torch

    if not c:
        return
    gap = c0 - a
    f = torch.as_tensor(inv_freq).float()
    angle = -gap * f
    emb = torch.cat((angle, angle))
    cos, sin = emb.cos(), emb.sin()
    half = f.numel()
    for kb, vb in zip(kbufs, vbufs):
        keys = kb[..., c0:c0 + c, :]
        if gap:
            kf = keys.float()
            rot = torch.cat((-kf[..., half:], kf[..., :half]), dim=-1)
            kb[..., a:a + c, :] = (kf * cos + rot * sin).to(keys.dtype)
        else:
            kb[..., a:a + c, :] = keys.clone()
        vb[..., a:a + c, :] = vb[..., c0:c0 + c, :].clone()
