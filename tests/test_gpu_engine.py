"""Drop-in through transformers on the GPU: a small random Qwen3 (head_dim 128,
8 query heads over 2 KV heads, fp16) run with the registered "threadcut"
attention and the GrowingLayer cache, against stock SDPA.

Mirrors the reference's engine tests (threadcut's tests/test_core.py): T3's
decode-equals-stock-transformers check, compared here on teacher-forced logits
(a random model's near-ties make greedy tokens a fragile oracle), and T2's
splice-equals-fresh-compute check with the reference's 3e-2 fp16 tolerance.
"""
import numpy as np
import pytest
import torch
from transformers import AutoModelForCausalLM, DynamicCache, Qwen3Config

from oracle import splice as osp
from threadcut_amd import attention, kv
from threadcut_amd.match import Split, split

pytestmark = pytest.mark.gpu

ATOL = 3e-2


@pytest.fixture(scope="module")
def model(gpu):
    torch.manual_seed(0)
    cfg = Qwen3Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=128, max_position_embeddings=4096,
                      rope_theta=1e6)
    m = AutoModelForCausalLM.from_config(cfg, dtype=torch.float16, attn_implementation=attention.NAME)
    return m.to(gpu).eval()


def rand_ids(n, seed, vocab=500):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(10, vocab, (n,), generator=g).tolist()


def run(m, ids, cache, impl, start=None):
    m.set_attn_implementation(impl)
    x = torch.tensor([ids], device=m.device)
    kw = {}
    if start is not None:
        kw["position_ids"] = torch.arange(start, start + len(ids), device=m.device)[None]
    return m(input_ids=x, past_key_values=cache, use_cache=True, **kw).logits[0, -1].float()


def kv_alone(m, ids, start):
    """KV of `ids` at positions start.. with no other context visible (stock SDPA)."""
    cache = DynamicCache(config=m.config)
    run(m, ids, cache, "sdpa", start)
    return cache


@torch.no_grad()
def test_decode_steps_match_stock_sdpa(model):
    """Prefill 40 tokens, then 12 single-token steps: every step's logits vs stock SDPA."""
    ids = rand_ids(52, 5)
    ours = kv.new_cache(model.config)
    ref = DynamicCache(config=model.config)
    run(model, ids[:40], ours, attention.NAME)
    run(model, ids[:40], ref, "sdpa")
    for t in ids[40:]:
        a = run(model, [t], ours, attention.NAME)
        b = run(model, [t], ref, "sdpa")
        assert (a - b).abs().max().item() <= ATOL
    assert ours.get_seq_length() == 52


@torch.no_grad()
def test_splice_matches_fresh_compute(model):
    """T2: cache A·B·C (each span computed alone) spliced to A·C, then D and one decode step."""
    A, B, C, D = rand_ids(9, 1), rand_ids(13, 2), rand_ids(11, 3), rand_ids(5, 4)
    inv = model.model.rotary_emb.inv_freq
    fresh = kv_alone(model, A, 0)
    c_alone = kv_alone(model, C, len(A))
    for lo, li in zip(fresh.layers, c_alone.layers):
        lo.keys = torch.cat((lo.keys, li.keys), 2)
        lo.values = torch.cat((lo.values, li.values), 2)
    ref_logits = run(model, D, fresh, "sdpa")

    cache = kv.new_cache(model.config)
    for span, start in ((A, 0), (B, len(A)), (C, len(A) + len(B))):
        part = kv_alone(model, span, start)
        for layer, p in zip(cache.layers, part.layers):
            layer.update(p.keys, p.values)
    s = split(A + B + C, A + C + D, min_suffix=4)
    assert s == Split(len(A), len(A) + len(B), len(C))
    kv.splice(cache, s, inv)
    assert cache.get_seq_length() == len(A) + len(C)
    logits = run(model, D, cache, attention.NAME)
    assert (logits - ref_logits).abs().max().item() <= ATOL

    # One decode step on the spliced cache goes through the HIP decode kernel.
    nxt = int(ref_logits.argmax())
    got = run(model, [nxt], cache, attention.NAME)
    want = run(model, [nxt], fresh, "sdpa")
    assert (got - want).abs().max().item() <= ATOL


@torch.no_grad()
def test_fused_append_cache_matches_plain_cache(model):
    """new_cache(fused_append=True): the attention kernel writes each decode token's K/V
    while it attends; logits and cache contents equal the copying cache's."""
    ids = rand_ids(30, 7)
    fused = kv.new_cache(model.config, fused_append=True)
    plain = kv.new_cache(model.config)
    ref = DynamicCache(config=model.config)
    for cache, impl in ((fused, attention.NAME), (plain, attention.NAME), (ref, "sdpa")):
        run(model, ids[:20], cache, impl)
    for t in ids[20:]:
        a = run(model, [t], fused, attention.NAME)
        b = run(model, [t], plain, attention.NAME)
        c = run(model, [t], ref, "sdpa")
        # The new token is attended in its own tile, so the fp32 summation order differs slightly.
        assert (a - b).abs().max().item() <= ATOL
        assert (a - c).abs().max().item() <= ATOL
    torch.cuda.synchronize()
    for i, (lf, lp) in enumerate(zip(fused.layers, plain.layers)):
        assert lf.pending is None and lf.n == lp.n == 30
        if i == 0:
            # Layer 0's K/V depend on the token embeddings alone: the rows the kernel wrote
            # are the rows the copying cache holds, bit for bit.
            assert torch.equal(lf.keys, lp.keys) and torch.equal(lf.values, lp.values)
        else:
            # Deeper layers see attention outputs, which differ in summation order.
            assert (lf.keys - lp.keys).abs().max().item() <= ATOL
            assert (lf.values - lp.values).abs().max().item() <= ATOL
    # A splice after fused appends sees every row the kernel wrote: it matches the
    # oracle's splice of the cache as it stood.
    s = Split(4, 9, 11)
    inv = model.model.rotary_emb.inv_freq
    before = [(lf.keys.cpu().numpy(), lf.values.cpu().numpy()) for lf in fused.layers]
    kv.splice(fused, s, inv)
    cos, sin = osp.rope_table(-s.gap, inv)
    for lf, (k0, v0) in zip(fused.layers, before):
        kw, vw, n = osp.splice_growing(k0, v0, 30, s.a, s.c0, s.c, cos, sin)
        assert lf.n == n == s.a + s.c
        assert np.array_equal(lf.keys.cpu().numpy(), kw[..., :n, :])
        assert np.array_equal(lf.values.cpu().numpy(), vw[..., :n, :])


@torch.no_grad()
def test_slab_cache_matches_per_layer_buffers(model):
    """new_cache(slab=True): every layer's buffers are views of one [L, 2, B, Hkv, cap, D]
    allocation. Prefill, fused-append decode steps across a capacity growth, a splice (one
    tc_splice_rope over the slab's views) and a captured decode step give the per-layer cache's
    results: bit-identical cache rows, identical logits."""
    from threadcut_amd.graph import DecodeGraph

    ids = rand_ids(2100, 8)
    slab = kv.new_cache(model.config, fused_append=True, slab=True)
    per = kv.new_cache(model.config, fused_append=True)
    a = run(model, ids[:2040], slab, attention.NAME)
    b = run(model, ids[:2040], per, attention.NAME)
    assert torch.equal(a, b)
    store = slab.layers[0].slab.tensor
    assert store.shape[:2] == (2, 2) and store.shape[-2] == 2048
    for i, layer in enumerate(slab.layers):
        assert layer.kbuf.data_ptr() == store[i, 0].data_ptr() and layer.vbuf.data_ptr() == store[i, 1].data_ptr()
    for t in ids[2040:2060]:  # crosses capacity 2048: the slab grows once for both layers
        a = run(model, [t], slab, attention.NAME)
        b = run(model, [t], per, attention.NAME)
        assert torch.equal(a, b)
    grown = slab.layers[0].slab.tensor
    assert grown.shape[-2] > 2048 and all(l.kbuf.data_ptr() == grown[i, 0].data_ptr()
                                         for i, l in enumerate(slab.layers))
    inv = model.model.rotary_emb.inv_freq
    s = kv.Split(100, 700, 1300)
    kv.splice(slab, s, inv)
    kv.splice(per, s, inv)
    for ls, lp in zip(slab.layers, per.layers):
        assert torch.equal(ls.keys, lp.keys) and torch.equal(ls.values, lp.values)
    dg_s = DecodeGraph(model, slab, max_new_tokens=4)
    dg_p = DecodeGraph(model, per, max_new_tokens=4)
    for t in ids[2060:2064]:
        a = dg_s.step([t]).float().clone()
        b = dg_p.step([t]).float().clone()
        torch.cuda.synchronize()
        assert torch.equal(a, b)
    dg_s.close()
    dg_p.close()
    for ls, lp in zip(slab.layers, per.layers):
        assert torch.equal(ls.keys, lp.keys)
