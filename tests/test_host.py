"""Host-side logic on the CPU: the Split rule, cache bookkeeping, the rotation
table, the prefill branch and the GPU-only guards of the hot path."""
import itertools
import random

import numpy as np
import pytest
import torch
from transformers import Qwen3Config

from oracle import match as oracle_match
from oracle import splice as osp
from threadcut_amd import attention, flash_decode, kv, workloads
from threadcut_amd.match import Split, lcp, split


def test_split_rule_known_answers():
    """The reference's test_split_rule (tests/test_core.py:59-64)."""
    A, B, C, D = [1, 2, 3], [7, 7], [4, 5, 6, 8, 9], [10, 11]
    assert split(A + B + C, A + C + D, min_suffix=3) == Split(3, 5, 5)
    assert split(A + B + C, A + C + D, min_suffix=3, suffix=False) == Split(3, 3, 0)
    assert split(A + C, A + C + D, min_suffix=3) == Split(8, 8, 0)
    assert split(A + C, A + C, min_suffix=3).a == len(A + C) - 1
    assert Split(3, 5, 5).gap == 2


def brute_split(cached, new, min_suffix, suffix=True):
    """The Split rule by exhaustive search: every start j > a and every run length
    c in [min_suffix, len(rest) - 1] with cached[j:j+c] == rest[:c]; first longest wins."""
    a = min(lcp(cached, new), len(new) - 1)
    rest = new[a:] if a >= 0 else []
    best = Split(a, a, 0)
    if not suffix or len(rest) <= min_suffix or len(cached) - (a + 1) < min_suffix:
        return best
    for j in range(a + 1, len(cached) - min_suffix + 1):
        runs = [c for c in range(min_suffix, len(rest)) if list(cached[j:j + c]) == list(rest[:c])]
        if runs and max(runs) > best.c:
            best = Split(a, j, max(runs))
    return best


def test_split_matches_exhaustive_search():
    rng = random.Random(0)
    for _ in range(400):
        vocab = rng.choice([2, 3, 5])
        cached = [rng.randrange(vocab) for _ in range(rng.randrange(0, 30))]
        new = cached[:rng.randrange(0, len(cached) + 1)] + [rng.randrange(vocab) for _ in range(rng.randrange(1, 12))]
        if rng.random() < 0.5 and len(cached) > 6:
            i = rng.randrange(len(cached) // 2)
            new = cached[:i] + cached[i + rng.randrange(1, 4):] + [rng.randrange(vocab)]
        for ms, sfx in itertools.product((1, 2, 4), (True, False)):
            want = Split(*oracle_match.split(cached, new, ms, sfx))
            assert split(cached, new, ms, sfx) == want
            assert brute_split(cached, new, ms, sfx) == want
            assert Split(*oracle_match.split_windows(cached, new, ms, sfx)) == want


def test_native_split_on_long_repetitive_caches():
    """The rolling-hash matcher against the oracle where windows repeat and hashes collide often."""
    rng = random.Random(1)
    for _ in range(30):
        period = rng.randrange(1, 6)
        unit = [rng.randrange(3) for _ in range(period)]
        cached = (unit * 400)[:rng.randrange(50, 1200)]
        cut = rng.randrange(0, len(cached))
        new = cached[:cut] + cached[cut + rng.randrange(1, 40):] + [7, 8]
        for ms in (1, 3, 8):
            assert split(cached, new, ms) == Split(*oracle_match.split(cached, new, ms))
    big = list(range(200000))
    s = split(big, big[:1000] + big[5000:150000], 32)
    assert s == Split(1000, 5000, 144999)


def test_lcp():
    assert lcp([], [1]) == 0
    assert lcp([1, 2, 3], [1, 2, 3]) == 3
    assert lcp([1, 2, 3], [1, 5]) == 1
    assert lcp(np.arange(5), np.arange(3)) == 3


def test_rope_table_is_the_oracle_table():
    inv = workloads.inv_freq(1e6)
    t = kv.rope_table(-6620, inv)
    cos, sin = osp.rope_table(-6620, inv)
    assert t.dtype == torch.float32 and t.shape == (128,)
    assert np.array_equal(t[:64].numpy(), cos) and np.array_equal(t[64:].numpy(), sin)


def test_inv_freq_matches_transformers():
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding

    rot = Qwen3RotaryEmbedding(Qwen3Config(head_dim=128, rope_theta=1e6))
    assert torch.equal(workloads.inv_freq(1e6), rot.inv_freq.float())


def test_rotate_half_and_repeat_kv():
    x = torch.arange(8.0).reshape(1, 1, 1, 8)
    assert kv.rotate_half(x).flatten().tolist() == [-4, -5, -6, -7, 0, 1, 2, 3]
    y = torch.randn(2, 3, 5, 4)
    r = attention.repeat_kv(y, 2)
    assert r.shape == (2, 6, 5, 4) and torch.equal(r[:, 1], y[:, 0]) and torch.equal(r[:, 4], y[:, 2])
    assert attention.repeat_kv(y, 1) is y


def test_growing_layer_bookkeeping_on_host_tensors():
    layer = kv.GrowingLayer()
    k = torch.randn(1, 8, 10, 128).half()
    keys, values = layer.update(k, k + 1)
    assert layer.n == 10 and layer.kbuf.shape[2] == 2048 and keys.shape[2] == 10
    assert layer.get_seq_length() == 10
    big = torch.randn(1, 8, 2100, 128).half()
    layer.update(big, big)
    assert layer.n == 2110 and layer.kbuf.shape[2] == max(2110, int(2048 * 1.25), 2048 + 2048)
    assert torch.equal(layer.keys[:, :, :10], k) and torch.equal(layer.values[:, :, :10], k + 1)
    layer.crop(7)
    assert layer.n == 7 and layer.keys.shape[2] == 7


def test_new_cache_has_growing_layers():
    cache = kv.new_cache(Qwen3Config(num_hidden_layers=3))
    assert len(cache.layers) == 3 and all(isinstance(layer, kv.GrowingLayer) for layer in cache.layers)


def test_kernel_entry_points_refuse_host_tensors():
    """The kernel wrappers (the reference's decode_attention is a GPU kernel too) refuse host
    tensors; the attention interface, shift_keys and splice run the reference's torch path for
    them instead (tests/test_cpu_path.py)."""
    q, k, v, _ = workloads.decode_inputs(0, n=32)
    with pytest.raises(RuntimeError, match="GPU"):
        flash_decode.decode_attention(q.reshape(8, 4, 128), k[0], v[0], 0.1)
    with pytest.raises(RuntimeError, match="GPU"):
        flash_decode.decode_attention_batched(q.reshape(1, 8, 4, 128), k, v, 0.1)
    layer = kv.GrowingLayer()
    layer.update(k, v)
    with pytest.raises(ValueError, match="past"):
        layer.splice(Split(2, 25, 10), workloads.inv_freq())


def test_decode_gate():
    """flash_decode.supports decides from the tensors alone which decode calls the kernels take."""
    q = torch.empty(1, 32, 1, 128, dtype=torch.float16)
    k = torch.empty(1, 8, 10, 128, dtype=torch.float16)
    assert not flash_decode.supports(q, k, k)  # host tensors
    assert not flash_decode.supports(q.float(), k.float(), k.float())


def test_prefill_branch_is_masked_sdpa():
    """q > 1 keeps the reference's prefill path: expanded KV and SDPA (threadcut/attention.py:43-46)."""
    g = torch.Generator().manual_seed(1)
    q = torch.randn(1, 8, 5, 16, generator=g)
    k = torch.randn(1, 2, 5, 16, generator=g)
    v = torch.randn(1, 2, 5, 16, generator=g)
    out, w = attention.attention(None, q, k, v, None, scaling=0.3)
    assert w is None and out.shape == (1, 5, 8, 16)
    kk = attention.repeat_kv(k, 4)
    vv = attention.repeat_kv(v, 4)
    s = (q @ kk.transpose(-1, -2)) * 0.3
    s = s + torch.triu(torch.full((5, 5), float("-inf")), 1)
    ref = (torch.softmax(s, -1) @ vv).transpose(1, 2)
    assert torch.allclose(out, ref, atol=1e-5)


def test_attention_is_registered():
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface

    assert attention.NAME == "threadcut"
    assert AttentionInterface._global_mapping[attention.NAME] is attention.attention
    assert attention.NAME in AttentionMaskInterface._global_mapping
