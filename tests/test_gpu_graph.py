"""Graph-captured decode on the GPU.

- ``tc_decode_append_attention_at`` (append position on the device) against
  the float64 oracle and against ``tc_decode_append_attention`` (host n),
  eagerly and replayed from one captured HIP graph whose own kernel advances
  the position: every replay attends one more token and writes its row.
- ``graph.DecodeGraph`` on a small random Qwen3 (head_dim 128, 8 q / 2 kv
  heads, fp16): every replayed step's logits against eager decoding with the
  same cache type (3e-2, the reference's fp16 tolerance for its model-level
  checks), the cache rows bit-exact where they do not depend on attention
  outputs (layer 0), and the cache usable eagerly after close().

The graphs are replayed several times with eager work and synchronizations
in between, and each replay is checked.
"""
import numpy as np
import pytest
import torch
from transformers import AutoModelForCausalLM, Qwen3Config

from oracle import decode as od
from threadcut_amd import attention, flash_decode, kv, workloads
from threadcut_amd.graph import DecodeGraph

pytestmark = pytest.mark.gpu

TOL = 2e-3
ATOL = 3e-2
SCALE = 128 ** -0.5


def ref64(q, k, v, n):
    """q [B,Hkv,G,D], k/v [B,Hkv,cap,D] (device) -> float64 over tokens [0, n)."""
    return od.attention_f64(q.float().cpu().numpy(), k[:, :, :n].float().cpu().numpy(),
                            v[:, :, :n].float().cpu().numpy(), SCALE)


@pytest.mark.parametrize("n0,cap", [(1, 64), (100, 300), (1500, 4096)])
def test_append_at_matches_host_position(gpu, n0, cap):
    """pos = n0 cached tokens: row n0 written, n0 + 1 tokens attended; same rows as the host-n entry."""
    g = torch.Generator(device=gpu)
    g.manual_seed(n0)
    b, hkv, grp, d = 2, 8, 4, 128
    kc = torch.randn((b, hkv, cap, d), generator=g, device=gpu).half()
    vc = torch.randn((b, hkv, cap, d), generator=g, device=gpu).half()
    q = torch.randn((b, hkv, grp, d), generator=g, device=gpu).half()
    kn = torch.randn((b, hkv, 1, d), generator=g, device=gpu).half()
    vn = torch.randn((b, hkv, 1, d), generator=g, device=gpu).half()
    k2, v2 = kc.clone(), vc.clone()
    pos = torch.full((b,), n0, dtype=torch.int32, device=gpu)
    print(f"case: append_at n0={n0} cap={cap}", flush=True)
    out = flash_decode.decode_append_at(q, kc, vc, kn, vn, pos, SCALE, torch.empty_like(q))
    out2 = flash_decode.decode_append_into(q, k2, v2, kn, vn, n0 + 1, SCALE, torch.empty_like(q))
    torch.cuda.synchronize()
    assert torch.equal(kc, k2) and torch.equal(vc, v2)
    assert torch.equal(kc[:, :, n0], kn[:, :, 0]) and torch.equal(vc[:, :, n0], vn[:, :, 0])
    want = ref64(q, kc, vc, n0 + 1)
    assert np.abs(out.float().cpu().numpy() - want).max() <= TOL
    assert np.abs(out2.float().cpu().numpy() - want).max() <= TOL


def test_append_at_per_sequence_positions(gpu):
    """Different positions per sequence (ragged batch), one of them at the last row."""
    g = torch.Generator(device=gpu)
    g.manual_seed(9)
    b, hkv, grp, d, cap = 3, 8, 4, 128, 700
    kc = torch.randn((b, hkv, cap, d), generator=g, device=gpu).half()
    vc = torch.randn((b, hkv, cap, d), generator=g, device=gpu).half()
    q = torch.randn((b, hkv, grp, d), generator=g, device=gpu).half()
    kn = torch.randn((b, hkv, 1, d), generator=g, device=gpu).half()
    vn = torch.randn((b, hkv, 1, d), generator=g, device=gpu).half()
    p = [0, 333, cap - 1]
    pos = torch.tensor(p, dtype=torch.int32, device=gpu)
    out = flash_decode.decode_append_at(q, kc, vc, kn, vn, pos, SCALE, torch.empty_like(q))
    torch.cuda.synchronize()
    for i, n0 in enumerate(p):
        assert torch.equal(kc[i, :, n0], kn[i, :, 0]) and torch.equal(vc[i, :, n0], vn[i, :, 0])
        want = ref64(q[i:i + 1], kc[i:i + 1], vc[i:i + 1], n0 + 1)
        assert np.abs(out[i:i + 1].float().cpu().numpy() - want).max() <= TOL


def test_append_at_graph_replays_advance(gpu):
    """One captured graph (append-attend, then pos += 1) replayed 6 times: replay r writes row
    n0 + r and attends n0 + r + 1 tokens; eager work and syncs between replays."""
    g = torch.Generator(device=gpu)
    g.manual_seed(3)
    b, hkv, grp, d, cap, n0 = 1, 8, 4, 128, 2048, 777
    kc = torch.randn((b, hkv, cap, d), generator=g, device=gpu).half()
    vc = torch.randn((b, hkv, cap, d), generator=g, device=gpu).half()
    q = torch.empty((b, hkv, grp, d), device=gpu).half()
    kn = torch.empty((b, hkv, 1, d), device=gpu).half()
    vn = torch.empty((b, hkv, 1, d), device=gpu).half()
    out = torch.empty_like(q)
    pos = torch.full((b,), n0, dtype=torch.int32, device=gpu)
    flash_decode.decode_append_at(q.normal_(), kc, vc, kn.normal_(), vn.normal_(), pos, SCALE, out)  # warm-up
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        flash_decode.decode_append_at(q, kc, vc, kn, vn, pos, SCALE, out)
        pos.add_(1)
    for r in range(6):
        q.copy_(torch.randn((b, hkv, grp, d), generator=g, device=gpu).half())
        kn.copy_(torch.randn((b, hkv, 1, d), generator=g, device=gpu).half())
        vn.copy_(torch.randn((b, hkv, 1, d), generator=g, device=gpu).half())
        graph.replay()
        torch.cuda.synchronize()
        print(f"case: replay {r}", flush=True)
        assert int(pos[0]) == n0 + r + 1
        assert torch.equal(kc[:, :, n0 + r], kn[:, :, 0]) and torch.equal(vc[:, :, n0 + r], vn[:, :, 0])
        want = ref64(q, kc, vc, n0 + r + 1)
        assert np.abs(out.float().cpu().numpy() - want).max() <= TOL


def test_layer_plans_sharing_a_workspace(gpu):
    """Six layers' DecodePlans on one workspace, captured as one graph and replayed three times with
    new queries between replays: every layer's output equals its own plan's on a private workspace,
    bit for bit, and the float64 closed form within the bar; a too-small workspace is refused."""
    g = torch.Generator(device=gpu)
    g.manual_seed(4)
    layers, n = 6, 1500
    qs = [torch.empty((1, 8, 4, 128), device=gpu).half() for _ in range(layers)]
    ks = [torch.randn((1, 8, n, 128), generator=g, device=gpu).half() for _ in range(layers)]
    vs = [torch.randn((1, 8, n, 128), generator=g, device=gpu).half() for _ in range(layers)]
    outs = [torch.empty_like(q) for q in qs]
    own = [torch.empty_like(q) for q in qs]
    shared = None
    plans = []
    for q, k, v, o in zip(qs, ks, vs, outs):
        plans.append(flash_decode.DecodePlan(q, k, v, SCALE, o, workspace=shared))
        shared = plans[-1].workspace
    privates = [flash_decode.DecodePlan(q, k, v, SCALE, o) for q, k, v, o in zip(qs, ks, vs, own)]
    assert all(p.workspace.data_ptr() == shared.data_ptr() for p in plans)
    for q in qs:
        q.normal_()
    for p in plans:
        p.run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for p in plans:
            p.run()
    for r in range(3):
        for q in qs:
            q.copy_(torch.randn(q.shape, generator=g, device=gpu).half())
        graph.replay()
        torch.cuda.synchronize()
        for p in privates:
            p.run()
        torch.cuda.synchronize()
        print(f"case: shared workspace, replay {r}", flush=True)
        for i in range(layers):
            assert torch.equal(outs[i], own[i]), i
            assert np.abs(outs[i].float().cpu().numpy() - ref64(qs[i], ks[i], vs[i], n)).max() <= TOL
    small = torch.empty(plans[0].workspace_bytes - 16, dtype=torch.uint8, device=gpu)
    with pytest.raises(ValueError):
        flash_decode.DecodePlan(qs[0], ks[0], vs[0], SCALE, outs[0], workspace=small)


@pytest.fixture(scope="module")
def model(gpu):
    torch.manual_seed(0)
    cfg = Qwen3Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=3,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=128, max_position_embeddings=4096,
                      rope_theta=1e6)
    m = AutoModelForCausalLM.from_config(cfg, dtype=torch.float16, attn_implementation=attention.NAME)
    return m.to(gpu).eval()


def ids_of(n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(10, 500, (n,), generator=g).tolist()


@torch.no_grad()
def test_decode_graph_matches_eager(model):
    dev = model.device
    ids = ids_of(40, 11)
    prompt, steps = ids[:25], ids[25:]
    caches = [kv.new_cache(model.config, fused_append=True) for _ in range(2)]
    for c in caches:
        model(input_ids=torch.tensor([prompt], device=dev), past_key_values=c, use_cache=True)
    eager = []
    for t in steps:
        eager.append(model(input_ids=torch.tensor([[t]], device=dev), past_key_values=caches[0],
                           use_cache=True).logits[0, -1].float().clone())
    dg = DecodeGraph(model, caches[1], max_new_tokens=len(steps))
    for i, t in enumerate(steps):
        got = dg.step(torch.tensor([t], device=dev))[0].float().clone()
        torch.cuda.synchronize()
        print(f"case: graph step {i}", flush=True)
        assert (got - eager[i]).abs().max().item() <= ATOL
        assert dg.n == 25 + i + 1
    dg.close()
    for i, (le, lg) in enumerate(zip(caches[0].layers, caches[1].layers)):
        le.flush()
        assert lg.n == le.n == 40 and lg.keys.shape[2] == 40
        if i == 0:
            assert torch.equal(le.keys, lg.keys) and torch.equal(le.values, lg.values)
        else:
            assert (le.keys - lg.keys).abs().max().item() <= ATOL
    # after close() the cache decodes eagerly again, continuing from 40 tokens
    nxt = ids_of(1, 12)
    a = model(input_ids=torch.tensor([nxt], device=dev), past_key_values=caches[0], use_cache=True).logits[0, -1]
    b = model(input_ids=torch.tensor([nxt], device=dev), past_key_values=caches[1], use_cache=True).logits[0, -1]
    assert (a.float() - b.float()).abs().max().item() <= ATOL
    assert caches[1].get_seq_length() == 41


@torch.no_grad()
def test_decode_graph_capacity_guard(model):
    dev = model.device
    cache = kv.new_cache(model.config)
    model(input_ids=torch.tensor([ids_of(10, 13)], device=dev), past_key_values=cache, use_cache=True)
    dg = DecodeGraph(model, cache, max_new_tokens=4)
    spare = dg.capacity - dg.n
    for t in ids_of(spare, 14):
        dg.step([t])
    with pytest.raises(RuntimeError, match="holds"):
        dg.step([1])
    dg.close()
    assert cache.layers[0].n == dg.capacity


@torch.no_grad()
def test_decode_graph_refuses_changes_outside_the_graph(model):
    """While a DecodeGraph holds the cache, splice, crop and eager updates raise (the captured
    kernels hold the buffers' addresses and the device position); a layer changed behind the
    graph's back stops step(); after close() the cache splices and decodes again."""
    dev = model.device
    cache = kv.new_cache(model.config, fused_append=True)
    model(input_ids=torch.tensor([ids_of(30, 15)], device=dev), past_key_values=cache, use_cache=True)
    dg = DecodeGraph(model, cache, max_new_tokens=4)
    dg.step([5])
    inv = model.model.rotary_emb.inv_freq
    with pytest.raises(RuntimeError, match="DecodeGraph holds"):
        kv.splice(cache, kv.Split(5, 10, 20), inv)
    with pytest.raises(RuntimeError, match="DecodeGraph holds"):
        cache.layers[1].crop(10)
    with pytest.raises(RuntimeError, match="DecodeGraph holds"):
        model(input_ids=torch.tensor([[7]], device=dev), past_key_values=cache, use_cache=True)
    assert dg.n == 31
    dg.step([6])
    cache.layers[2].n -= 1  # a change the graph cannot see
    with pytest.raises(RuntimeError, match="changed outside"):
        dg.step([7])
    cache.layers[2].n += 1
    dg.close()
    with pytest.raises(RuntimeError, match="closed"):
        dg.step([8])
    kv.splice(cache, kv.Split(5, 10, 22), inv)
    assert cache.get_seq_length() == 27
    out = model(input_ids=torch.tensor([[9]], device=dev), past_key_values=cache, use_cache=True).logits
    assert bool(torch.isfinite(out).all()) and cache.get_seq_length() == 28
