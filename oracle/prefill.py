"""Oracle of the prefill attention — TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Functions and the reference lines each restates:

- ``repeat_kv``: threadcut/attention.py:25-27 (each KV head repeated g times,
  head index h*g + i).
- ``prefill_f64``: the prefill branch of threadcut/attention.py:43-47 in
  float64 numpy — scores q·kᵀ·scale against the expanded K/V, the boolean
  mask (False = -inf) or SDPA's is_causal triangle (key j visible to query t
  iff j <= t + n - q; with q == n, which is when the reference sets
  is_causal, this is torch's upper-left triangle), softmax, times V, output
  [b, q, hq, d]. A query row with no visible key yields zeros.
- ``sdpa_reference``: the same branch as the reference runs it on the CPU:
  repeat_kv + torch SDPA (a library routine), transposed to [b, q, hq, d].

Pins (tests/test_oracle_prefill.py): ``prefill_f64`` against torch SDPA in
float64 (a library routine) for masked, causal and unmasked calls;
brute-force loops on tiny shapes; closed forms that a wrong index breaks —
one visible key returns that key's value row, constant V returns that row,
q = 0 returns the mean of the visible V rows, the first causal query sees
only key 0; an all-True mask equals no mask; and mutated copies (mask
transposed, heads mapped h + i*hkv, causal triangle off by one) fail them.
"""
import numpy as np


def repeat_kv(x, g):
    """[b, h, s, d] -> [b, h*g, s, d], head h*g + i = head h."""
    return np.repeat(np.asarray(x), g, axis=1)


def visible(q_len, n, mask=None, causal=False, batch=1):
    """Boolean [b, q, n] of the keys each query row may attend to."""
    if mask is not None:
        m = np.asarray(mask, bool)
        if m.ndim == 4:
            m = m[:, 0]
        return np.broadcast_to(m, (batch, q_len, n))
    if causal:
        t = np.arange(q_len)[:, None] + (n - q_len)
        return np.broadcast_to(np.arange(n)[None, :] <= t, (batch, q_len, n))
    return np.ones((batch, q_len, n), bool)


def prefill_f64(q, k, v, scale, mask=None, causal=False):
    """q [b, hq, L, d], k/v [b, hkv, n, d] -> float64 [b, L, hq, d]."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    b, hq, L, d = q.shape
    g = hq // k.shape[1]
    n = k.shape[2]
    kk, vv = repeat_kv(k, g), repeat_kv(v, g)
    s = np.einsum("bhtd,bhjd->bhtj", q, kk) * scale
    vis = visible(L, n, mask, causal, b)[:, None]
    s = np.where(vis, s, -np.inf)
    m = s.max(-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.where(vis, np.exp(s - m), 0.0)
    den = p.sum(-1, keepdims=True)
    p = p / np.where(den > 0, den, 1.0)
    out = np.einsum("bhtj,bhjd->bhtd", p, vv)
    return out.transpose(0, 2, 1, 3)


def sdpa_reference(query, key, value, mask, scale):
    """threadcut/attention.py:43-47 on torch CPU tensors (float32 or float64)."""
    import torch
    import torch.nn.functional as F

    b, hq, L, d = query.shape
    g = hq // key.shape[1]
    kk = key.repeat_interleave(g, dim=1)
    vv = value.repeat_interleave(g, dim=1)
    is_causal = mask is None and L > 1 and L == key.shape[2]
    out = F.scaled_dot_product_attention(query, kk, vv, attn_mask=mask, scale=scale, is_causal=is_causal)
    return out.transpose(1, 2)
