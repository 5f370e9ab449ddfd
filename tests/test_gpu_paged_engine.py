"""The paged cache as the engine's cache, on the GPU.

- ``PagedKV.prefill`` (tc_prefill_paged_attention): the prefill branch of
  threadcut/attention.py:43-46 reading K/V from page pools through per-token
  row offsets, against the float64 oracle on the gathered keys (max-abs 2e-3
  fp16, 1.6e-2 bf16, as the contiguous prefill), with pages handed out from a
  shuffled free list and prunes that leave fragments starting mid-tile.
- ``paged.new_paged_cache`` through transformers with the "threadcut"
  attention: prefill chunks, decode steps with the fused append, a splice
  (prune), and the decode step captured as a HIP graph, against the
  GrowingLayer cache and stock SDPA (3e-2, the reference's fp16 tolerance for
  model-level checks).
"""
import random

import numpy as np
import pytest
import torch
from transformers import AutoModelForCausalLM, DynamicCache, Qwen3Config

from oracle import prefill as opf
from threadcut_amd import attention, kv, paged, prefill, workloads
from threadcut_amd.graph import DecodeGraph
from threadcut_amd.match import Split, split

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5
ATOL = 3e-2


def paged_with(dev, layers, n, page_tokens, seed, dtype=torch.float16, hkv=8, prune=None):
    """A one-sequence PagedKV holding n tokens (appended in random chunks from a shuffled
    free list; optionally pruned with `prune` from n + gap tokens) and its keys/values in
    logical order on the host, per layer [Hkv, n, D]."""
    rnd = random.Random(seed)
    total = n if prune is None else prune.c0 + prune.c
    pages = -(-total // page_tokens) * 2 + 8
    cache = paged.PagedKV(layers, hkv, pages, page_tokens, dtype=dtype, device=dev)
    rnd.shuffle(cache.table.free)
    g = torch.Generator().manual_seed(seed)
    host = [(torch.randn(hkv, total, 128, generator=g).to(dtype), torch.randn(hkv, total, 128, generator=g).to(dtype))
            for _ in range(layers)]
    done = 0
    while done < total:
        m = min(total - done, rnd.choice([1, 5, 16, 17, 64, 300]))
        cache.append(0, [host[l][0][:, done:done + m].to(dev) for l in range(layers)],
                     [host[l][1][:, done:done + m].to(dev) for l in range(layers)])
        done += m
    if prune is not None:
        cache.prune(0, prune, workloads.inv_freq())
    kept = [cache.gather(l) for l in range(layers)]
    assert cache.length() == n
    return cache, [(k.cpu(), v.cpu()) for k, v in kept]


@pytest.mark.parametrize("g", [1, 2, 4, 8])
@pytest.mark.parametrize("page_tokens,n,q,mode", [(64, 700, 700, "causal"), (16, 333, 100, "mask"),
                                                   (48, 1200, 64, "none"), (64, 2100, 300, "mask")])
def test_paged_prefill_matches_oracle(gpu, g, page_tokens, n, q, mode):
    hkv = 8 if g <= 4 else 4
    cache, kvs = paged_with(gpu, 1, n, page_tokens, 100 + g + n, hkv=hkv)
    gq = torch.Generator().manual_seed(7 + n)
    query = torch.randn(1, hkv * g, q, 128, generator=gq).half()
    mask = None
    if mode == "mask":
        vis = torch.rand(q, n, generator=gq) < 0.7
        vis[:, -q:] &= torch.ones(q, q, dtype=torch.bool).tril()
        mask = vis[None, None]
    print(f"case: paged prefill g={g} P={page_tokens} n={n} q={q} {mode}", flush=True)
    out = cache.prefill(0, query.to(gpu).transpose(1, 2).contiguous().transpose(1, 2), SCALE,
                        None if mask is None else mask.to(gpu), causal=mode == "causal")
    torch.cuda.synchronize()
    k, v = kvs[0]
    want = opf.prefill_f64(query.float().numpy(), k[None].float().numpy(), v[None].float().numpy(), SCALE,
                           mask=None if mask is None else mask.numpy(), causal=mode == "causal")
    assert np.abs(out.float().cpu().numpy() - want).max() <= 2e-3


@pytest.mark.parametrize("page_tokens", [64, 16])
@pytest.mark.parametrize("q,mode", [(200, "causal"), (1000, "causal"), (300, "mask"), (64, "none")])
def test_paged_prefill_bit_identical_to_contiguous(gpu, page_tokens, q, mode):
    """The paged and the contiguous prefill run the same arithmetic and differ only in where a
    row is read from. With 64-token pages filled in order every full 64-key tile is one page's
    consecutive rows (addressed from its first offset), with 16-token pages every tile gathers
    its rows through the per-token offsets, and the last, partial tile (1000 keys) gathers in
    both: each must give the contiguous kernel's output bit for bit."""
    n = 1000
    cache, kvs = paged_with(gpu, 1, n, page_tokens, 41 + q)
    gq = torch.Generator().manual_seed(q)
    query = torch.randn(1, 32, q, 128, generator=gq).half().to(gpu)
    mask = None
    if mode == "mask":
        vis = torch.rand(q, n, generator=gq) < 0.7
        vis[:, -q:] &= torch.ones(q, q, dtype=torch.bool).tril()
        mask = vis[None, None].to(gpu)
    print(f"case: paged vs contiguous prefill P={page_tokens} q={q} {mode}", flush=True)
    got = cache.prefill(0, query, SCALE, mask, causal=mode == "causal")
    k, v = kvs[0]
    want = prefill.prefill_attention(query, k[None].to(gpu), v[None].to(gpu), mask, SCALE,
                                     is_causal=mode == "causal")
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("s", [Split(37, 100, 1000), Split(5, 600, 63), Split(0, 17, 500)])
def test_paged_prefill_after_prunes_bf16(gpu, s):
    """Prunes leave fragments that start mid-tile and mid-page; the keys keep their logical order."""
    n = s.a + s.c
    cache, kvs = paged_with(gpu, 2, n, 64, 300 + s.c0, dtype=torch.bfloat16, prune=s)
    query = torch.randn(1, 32, 40, 128, generator=torch.Generator().manual_seed(s.c)).bfloat16()
    print(f"case: paged prefill after {s} bf16", flush=True)
    for layer in range(2):
        out = cache.prefill(layer, query.to(gpu), SCALE, causal=True)
        torch.cuda.synchronize()
        k, v = kvs[layer]
        want = opf.prefill_f64(query.float().numpy(), k[None].float().numpy(), v[None].float().numpy(), SCALE,
                               causal=True)
        assert np.abs(out.float().cpu().numpy() - want).max() <= 1.6e-2


@pytest.fixture(scope="module")
def model(gpu):
    torch.manual_seed(0)
    cfg = Qwen3Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=3,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=128, max_position_embeddings=4096,
                      rope_theta=1e6)
    m = AutoModelForCausalLM.from_config(cfg, dtype=torch.float16, attn_implementation=attention.NAME)
    return m.to(gpu).eval()


def ids_of(n, seed):
    return torch.randint(10, 500, (n,), generator=torch.Generator().manual_seed(seed)).tolist()


def run(m, ids, cache, impl=attention.NAME, start=None):
    m.set_attn_implementation(impl)
    kw = {}
    if start is not None:
        kw["position_ids"] = torch.arange(start, start + len(ids), device=m.device)[None]
    return m(input_ids=torch.tensor([ids], device=m.device), past_key_values=cache, use_cache=True,
             **kw).logits[0, -1].float()


@torch.no_grad()
def test_paged_cache_matches_growing_cache(model):
    """Prefill in chunks, then fused-append decode steps: the paged cache gives the logits of the
    GrowingLayer cache and of stock SDPA; its pages hold exactly the rows the GrowingLayer holds
    for layer 0 (whose K/V depend on the token embeddings alone)."""
    ids = ids_of(260, 21)
    pc = paged.new_paged_cache(model.config, num_pages=64, page_tokens=16)
    gc = kv.new_cache(model.config, fused_append=True)
    ref = DynamicCache(config=model.config)
    for lo in range(0, 200, 70):
        a = run(model, ids[lo:min(lo + 70, 200)], pc)
        b = run(model, ids[lo:min(lo + 70, 200)], gc)
        c = run(model, ids[lo:min(lo + 70, 200)], ref, "sdpa")
        assert (a - b).abs().max().item() <= ATOL and (a - c).abs().max().item() <= ATOL
    for i, t in enumerate(ids[200:]):
        a = run(model, [t], pc)
        b = run(model, [t], gc)
        c = run(model, [t], ref, "sdpa")
        print(f"case: paged decode step {i}", flush=True)
        assert (a - b).abs().max().item() <= ATOL and (a - c).abs().max().item() <= ATOL
    assert pc.get_seq_length() == 260
    state = paged.state_of(pc)
    k, v = state.kv.gather(0)
    gc.layers[0].flush()
    assert torch.equal(k, gc.layers[0].keys[0]) and torch.equal(v, gc.layers[0].values[0])


@torch.no_grad()
def test_dropped_paged_caches_free_their_pools(model):
    """A server makes a fresh cache whenever a turn cannot be spliced (threadcut/engine.py:55):
    paged caches that nothing holds any more give their pools back (the layer registry holds
    its entries weakly), so device memory returns to where it started."""
    import gc

    ids = ids_of(150, 23)

    def turn(i):
        pc = paged.new_paged_cache(model.config, num_pages=64, page_tokens=16)
        run(model, ids[:120], pc)
        run(model, [ids[120 + i]], pc)
        assert paged.state_of(pc).kv is not None

    turn(0)  # warm-up: whatever the forward allocates once
    gc.collect()
    torch.cuda.synchronize()
    start, registered = torch.cuda.memory_allocated(), len(paged._LAYERS)
    for i in range(1, 5):
        turn(i)
    gc.collect()
    torch.cuda.synchronize()
    assert len(paged._LAYERS) == registered
    assert torch.cuda.memory_allocated() == start


@torch.no_grad()
def test_paged_splice_matches_fresh_compute(model):
    """T2 on the paged cache: A·B·C (each span computed alone) pruned to A·C by kv.splice (pages
    of B freed, C's keys re-rotated in place), then D and two decode steps, against a fresh
    computation of A, then C placed after A (stock SDPA)."""
    A, B, C, D = ids_of(40, 1), ids_of(77, 2), ids_of(150, 3), ids_of(9, 4)
    inv = model.model.rotary_emb.inv_freq
    fresh = DynamicCache(config=model.config)
    run(model, A, fresh, "sdpa")
    c_alone = DynamicCache(config=model.config)
    run(model, C, c_alone, "sdpa", start=len(A))
    for lo, li in zip(fresh.layers, c_alone.layers):
        lo.keys, lo.values = torch.cat((lo.keys, li.keys), 2), torch.cat((lo.values, li.values), 2)
    pc = paged.new_paged_cache(model.config, num_pages=40, page_tokens=16)
    for span, start in ((A, 0), (B, len(A)), (C, len(A) + len(B))):
        part = DynamicCache(config=model.config)
        run(model, span, part, "sdpa", start=start)
        for layer, p in zip(pc.layers, part.layers):
            layer.update(p.keys, p.values)
    free_before = len(paged.state_of(pc).kv.table.free)
    s = split(A + B + C, A + C + D, min_suffix=4)
    assert s == Split(len(A), len(A) + len(B), len(C))
    kv.splice(pc, s, inv)
    assert pc.get_seq_length() == len(A) + len(C)
    assert len(paged.state_of(pc).kv.table.free) > free_before  # B's pages came back
    got = run(model, D, pc)
    want = run(model, D, fresh, "sdpa")
    assert (got - want).abs().max().item() <= ATOL
    for t in ids_of(2, 5):
        got = run(model, [t], pc)
        want = run(model, [t], fresh, "sdpa")
        assert (got - want).abs().max().item() <= ATOL


@torch.no_grad()
def test_paged_decode_graph_matches_eager(model):
    """The decode step over the paged cache captured once and replayed: slots reserved ahead,
    lengths advanced on the device. Every replay's logits against eager paged decoding; after
    close() the unused reservation is released and eager decoding continues."""
    ids = ids_of(80, 31)
    caches = [paged.new_paged_cache(model.config, num_pages=32, page_tokens=16) for _ in range(2)]
    for c in caches:
        run(model, ids[:50], c)
    eager = [run(model, [t], caches[0]).clone() for t in ids[50:70]]
    state = paged.state_of(caches[1])
    dg = DecodeGraph(model, caches[1], max_new_tokens=20)
    with pytest.raises(RuntimeError, match="DecodeGraph holds"):
        kv.splice(caches[1], Split(5, 10, 20), model.model.rotary_emb.inv_freq)
    for i, t in enumerate(ids[50:70]):
        got = dg.step([t])[0].float().clone()
        torch.cuda.synchronize()
        print(f"case: paged graph step {i}", flush=True)
        assert (got - eager[i]).abs().max().item() <= ATOL
    dg.close()
    assert state.kv.table.length(0) == 70 == caches[1].get_seq_length()
    k0, v0 = paged.state_of(caches[0]).kv.gather(0)
    k1, v1 = state.kv.gather(0)
    assert torch.equal(k0, k1) and torch.equal(v0, v1)  # layer 0's rows, written by the captured kernels
    a = run(model, [ids[70]], caches[0])
    b = run(model, [ids[70]], caches[1])
    assert (a - b).abs().max().item() <= ATOL
