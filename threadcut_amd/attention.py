"""GQA-aware attention registered into transformers as ``"threadcut"``.

Drop-in for threadcut/attention.py:22-51. Decode (one query token, no mask):
the g query heads sharing a KV head are handed to the split-KV HIP kernels of
``flash_decode`` together with the unexpanded cache views, for any batch
size (the reference used its GPU kernel for b == 1 and SDPA otherwise; both
compute the same softmax), whenever the kernels take the tensors
(``flash_decode.supports``: GPU, float16/bfloat16, head_dim 128, g <= 8).
Other decode calls, host tensors included, keep the reference's own decode
path for them (threadcut/attention.py:40-42): SDPA with each group's query
heads folded into a length-g query against the unexpanded cache. Prefill
(threadcut/attention.py:43-46) runs the GQA-native HIP kernel of ``prefill``
on the unexpanded K/V for GPU tensors in float16/bfloat16 with head_dim 128,
g in (1, 2, 4, 8) and no mask or a boolean [b|1, 1, q, n] mask (what the
registered ``sdpa_mask`` produces). Other prefill calls keep the reference's
own path: expand KV once and run SDPA. A paged cache (``paged.new_paged_cache``)
hands over its page pools; its layers run the paged decode and prefill kernels.
"""
import torch
import torch.nn.functional as F
from transformers import AttentionInterface
from transformers.masking_utils import AttentionMaskInterface, sdpa_mask

from . import kv, paged, prefill
from .flash_decode import decode_append_at, decode_append_into, decode_into, supports as decode_supports

NAME = "threadcut"


def repeat_kv(x, n):
    """[b, h, s, d] -> [b, h*n, s, d], each KV head repeated n times in place order."""
    if n == 1:
        return x
    b, h, s, d = x.shape
    return x.unsqueeze(2).expand(b, h, n, s, d).reshape(b, h * n, s, d)


def attention(module, query, key, value, attention_mask, dropout=0.0, scaling=None, **kwargs):
    """transformers attention interface (threadcut/attention.py:30-47).

    query [b, hq, q, d] (usually a transposed view), key/value [b, hkv, n, d]
    (views into the cache). Returns ([b, q, hq, d] contiguous, None).
    """
    b, hq, q, d = query.shape
    scaling = scaling if scaling is not None else query.shape[-1] ** -0.5
    layer = paged.layer_of(key)
    if layer is not None:  # a paged cache layer handed over its pools
        return paged.attention(layer, query, attention_mask, scaling), None
    hkv = key.shape[1]
    g = hq // hkv
    if q == 1 and attention_mask is None and not decode_supports(query, key, value):
        # The reference's decode path for calls its GPU kernel does not serve
        # (attention.py:40-42): the g query heads of a KV head as a length-g query.
        pending = kv.take_pending(key)
        if pending is not None:
            pending.flush()
        out = F.scaled_dot_product_attention(query.reshape(b, hkv, g, d), key, value, scale=scaling)
        return out.reshape(b, hq, 1, d).transpose(1, 2).contiguous(), None
    if q == 1 and attention_mask is None:
        # [b, 1, hq, d] contiguous is [b, hkv, g, d] with head index h*g + i.
        out = torch.empty((b, 1, hq, d), dtype=query.dtype, device=query.device)
        layer = kv.take_pending(key)
        if layer is not None:
            # GrowingLayer deferred this token's append: write it and attend in one launch.
            k_new, v_new = layer.pending
            layer.pending = None
            if layer.device_pos is not None:  # graph-captured step: the position lives on the device
                decode_append_at(query.reshape(b, hkv, g, d), layer.kbuf, layer.vbuf, k_new, v_new,
                                 layer.device_pos, scaling, out.view(b, hkv, g, d))
            else:
                decode_append_into(query.reshape(b, hkv, g, d), layer.kbuf, layer.vbuf, k_new, v_new, layer.n,
                                   scaling, out.view(b, hkv, g, d))
        else:
            decode_into(query.reshape(b, hkv, g, d), key, value, scaling, out.view(b, hkv, g, d))
        return out, None
    pending = kv.take_pending(key)
    if pending is not None:  # a deferred append must land before SDPA reads the cache
        pending.flush()
    is_causal = attention_mask is None and q > 1 and q == key.shape[2]
    if prefill.supports(query, key, attention_mask):
        return prefill.prefill_attention(query, key, value, attention_mask, scaling, is_causal), None
    out = F.scaled_dot_product_attention(query, repeat_kv(key, g), repeat_kv(value, g),
                                         attn_mask=attention_mask, scale=scaling, is_causal=is_causal)
    return out.transpose(1, 2).contiguous(), None


AttentionInterface.register(NAME, attention)
AttentionMaskInterface.register(NAME, sdpa_mask)
