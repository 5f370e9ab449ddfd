"""Paged KV cache on the GPU: decode over the tile table against the float64
closed form on the gathered keys, and the prune (freed pages, the kept
suffix's keys rotated in place) bit-exact against the oracle's splice of the
same cache held contiguously."""
import random

import numpy as np
import pytest
import torch

from oracle import decode as od
from oracle import splice as osp
from threadcut_amd import _lib, workloads
from threadcut_amd.match import Split
from threadcut_amd.paged import PagedKV

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5
# Absolute bound, plus the output's own rounding: half an ulp of |result| in
# the storage dtype (bf16 keeps 8 significant bits, so an output of 2.67 rounds
# by up to 2^-7).
TOL = {torch.float16: 2e-3, torch.bfloat16: 4e-3}
HALF_ULP = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


def np_of(t):
    """fp16 as float16, bf16 as uint16 bits (the oracle's storage forms)."""
    t = t.detach().cpu().contiguous()
    return t.numpy() if t.dtype == torch.float16 else t.view(torch.int16).numpy().view(np.uint16)


def filled(dev, layers, lens, page_tokens, seed, dtype=torch.float16, hkv=8, slack=8):
    """A PagedKV whose sequences received their tokens in random chunks,
    interleaved, from a shuffled free list; returns (cache, host K/V per
    sequence and layer, [Hkv, n, D])."""
    rnd = random.Random(seed)
    pages = sum(-(-n // page_tokens) for n in lens) + slack
    cache = PagedKV(layers, hkv, pages, page_tokens, batch=len(lens), dtype=dtype, device=dev)
    rnd.shuffle(cache.table.free)
    g = torch.Generator().manual_seed(seed)
    host = [[(torch.randn(hkv, n, 128, generator=g).to(dtype), torch.randn(hkv, n, 128, generator=g).to(dtype))
             for _ in range(layers)] for n in lens]
    done = [0] * len(lens)
    while any(d < n for d, n in zip(done, lens)):
        b = rnd.choice([i for i in range(len(lens)) if done[i] < lens[i]])
        m = min(lens[b] - done[b], rnd.choice([1, 5, 16, 17, 64, 300, 2048]))
        sl = slice(done[b], done[b] + m)
        cache.append(b, [host[b][l][0][:, sl].to(dev) for l in range(layers)],
                     [host[b][l][1][:, sl].to(dev) for l in range(layers)])
        done[b] += m
    return cache, host


def closed_form(q, k, v):
    return od.attention_f64(q.float().numpy(), k.float().numpy(), v.float().numpy(), SCALE)


def check_decode(cache, layer, host_kv, g, seed, split=None):
    """Paged decode of one layer vs the closed form on host_kv[b] = (K, V)."""
    dt = cache.dtype
    q = torch.randn(cache.table.batch, cache.kv_heads, g, 128, generator=torch.Generator().manual_seed(seed)).to(dt)
    out = cache.decode(layer, q.to(cache.device), SCALE, split=split)
    torch.cuda.synchronize()
    for b, (k, v) in enumerate(host_kv):
        want = closed_form(q[b], k, v)
        excess = np.abs(out[b].float().cpu().numpy() - want) - (TOL[dt] + HALF_ULP[dt] * np.abs(want))
        assert excess.max() <= 0, f"sequence {b} ({k.shape[1]} tokens): error above the bound by {excess.max()}"


@pytest.mark.parametrize("page_tokens", [16, 64, 48])
@pytest.mark.parametrize("lens", [[1], [10240], [3000, 0, 17, 777]])
def test_paged_decode_matches_closed_form(gpu, page_tokens, lens):
    print(f"case: paged decode P={page_tokens} lens={lens}", flush=True)
    cache, host = filled(gpu, 1, lens, page_tokens, seed=page_tokens + len(lens))
    check_decode(cache, 0, [h[0] for h in host], 4, seed=3)


@pytest.mark.parametrize("g", [1, 2, 8])
def test_paged_decode_groups_and_bf16(gpu, g):
    print(f"case: paged decode g={g} bf16", flush=True)
    cache, host = filled(gpu, 1, [1500, 4100], 32, seed=g, dtype=torch.bfloat16)
    check_decode(cache, 0, [h[0] for h in host], g, seed=g)


def test_paged_decode_tiles_past_the_lane_preload(gpu):
    """One split of 10240 tokens: each wave walks 160 tiles, so tiles past the
    64th read their table entries from memory."""
    print("case: paged decode, one split over 10240 tokens", flush=True)
    cache, host = filled(gpu, 1, [10240], 64, seed=11)
    check_decode(cache, 0, [host[0][0]], 4, seed=12, split=10240)


def test_paged_decode_matches_contiguous_decode(gpu):
    """Same keys, paged and contiguous: the two HIP paths agree to rounding."""
    from threadcut_amd import flash_decode

    print("case: paged vs contiguous decode", flush=True)
    cache, host = filled(gpu, 1, [5000], 64, seed=21)
    q = torch.randn(1, 8, 4, 128, generator=torch.Generator().manual_seed(22)).half().to(gpu)
    k, v = (t.unsqueeze(0).to(gpu) for t in host[0][0])
    want = flash_decode.decode_into(q, k, v, SCALE, torch.empty_like(q))
    got = cache.decode(0, q, SCALE)
    torch.cuda.synchronize()
    assert (got.float() - want.float()).abs().max().item() <= 1e-3


def test_invalid_tile_entries_count_as_empty(gpu):
    """Entries with a page outside the pool, too many rows or slots past the
    page's end load nothing: the result equals the valid entries alone."""
    print("case: invalid tile entries", flush=True)
    cache, host = filled(gpu, 1, [300], 16, seed=31)
    tab, cnt = cache.table.tile_table()
    valid = tab[0, :cnt[0]]
    bad = np.array([[cache.table.num_pages, 0, 16, 0], [-1, 0, 4, 0], [0, 10, 8, 0], [0, 0, 17, 0], [0, -16, 4, 0]],
                   dtype=np.int32)
    mixed = np.concatenate([valid[:5], bad, valid[5:]])[None]
    q = torch.randn(1, 8, 4, 128, generator=torch.Generator().manual_seed(32)).half().to(gpu)
    lib = _lib.load()
    kp, vp = cache.k_pools[0], cache.v_pools[0]
    tdev = torch.from_numpy(mixed).to(gpu)
    cdev = torch.tensor([mixed.shape[1]], dtype=torch.int32, device=gpu)
    s = lib.tc_decode_num_splits(1, 8, 16 * mixed.shape[1], 0, 0)
    ws = torch.empty(lib.tc_decode_workspace_bytes(1, 8, 4, 128, s), dtype=torch.uint8, device=gpu)
    out = torch.empty_like(q)
    rc = lib.tc_decode_paged_attention(q.data_ptr(), _lib.i64x3(*q.stride()[:3]), kp.data_ptr(), vp.data_ptr(),
                                       _lib.i64x3(*kp.stride()[:3]), kp.shape[0], kp.shape[2], tdev.data_ptr(),
                                       cdev.data_ptr(), mixed.shape[1], 1, 8, 4, 128, _lib.TC_DTYPE_F16, SCALE, 0,
                                       ws.data_ptr(), ws.numel(), out.data_ptr(), _lib.i64x3(*out.stride()[:3]),
                                       _lib.stream_of(gpu))
    _lib.check(rc, "tc_decode_paged_attention")
    torch.cuda.synchronize()
    err = np.abs(out[0].float().cpu().numpy() - closed_form(q[0].cpu(), *host[0][0])).max()
    assert err <= 2e-3


def oracle_prune(k, v, s, inv, dtype):
    cos, sin = osp.rope_table(-s.gap, inv)
    name = "float16" if dtype == torch.float16 else "bfloat16"
    kb, vb, n = osp.splice_growing(np_of(k), np_of(v), k.shape[1], s.a, s.c0, s.c, cos, sin, name)
    return kb[:, :n], vb[:, :n], n


@pytest.mark.parametrize("page_tokens", [16, 64])
@pytest.mark.parametrize("s", [Split(10, 17, 20), Split(37, 1000, 2999), Split(100, 3000, 0), Split(0, 0, 50),
                               Split(5, 5, 100), Split(64, 128, 3872), Split(0, 3999, 1)])
def test_paged_prune_matches_contiguous_splice(gpu, page_tokens, s):
    n, layers = 4000, 3
    print(f"case: paged prune P={page_tokens} {s}", flush=True)
    cache, host = filled(gpu, layers, [n], page_tokens, seed=41)
    inv = workloads.inv_freq(1e6)
    used_before = set(range(cache.table.num_pages)) - set(cache.table.free)
    freed = cache.prune(0, s, inv)
    torch.cuda.synchronize()
    want = []
    for layer in range(layers):
        kb, vb, nn = oracle_prune(*host[0][layer], s, inv, cache.dtype)
        k, v = cache.gather(layer)
        assert cache.length() == nn
        assert np.array_equal(bits(k), kb.view(np.int16)), f"K layer {layer}"
        assert np.array_equal(bits(v), vb.view(np.int16)), f"V layer {layer}"
        want.append((kb, vb))
    # Exactly the pages no kept token uses went back to the free list.
    kept = set(cache.table.token_slots(0)[:, 0].tolist())
    assert set(freed) == used_before - kept
    assert len(freed) >= max(0, (s.c0 - s.a) // page_tokens - 1) + max(0, (n - s.c0 - s.c) // page_tokens - 1)
    # Decode on the pruned cache, then after more tokens are appended.
    check_decode(cache, 1, [tuple(torch.from_numpy(x) for x in want[1])], 4, seed=42)
    g = torch.Generator().manual_seed(43)
    extra = [(torch.randn(8, 70, 128, generator=g).half(), torch.randn(8, 70, 128, generator=g).half())
             for _ in range(layers)]
    cache.append(0, [e[0].to(gpu) for e in extra], [e[1].to(gpu) for e in extra])
    k2 = torch.cat([torch.from_numpy(want[2][0]), extra[2][0]], dim=1)
    v2 = torch.cat([torch.from_numpy(want[2][1]), extra[2][1]], dim=1)
    check_decode(cache, 2, [(k2, v2)], 4, seed=44)


def test_repeated_prunes_bf16(gpu):
    """Three prunes in a row on a bf16 cache, each checked against the oracle."""
    print("case: repeated paged prunes bf16", flush=True)
    cache, host = filled(gpu, 2, [3000], 64, seed=51, dtype=torch.bfloat16)
    inv = workloads.inv_freq(1e6)
    cur = [(np_of(k), np_of(v)) for k, v in host[0]]
    for s in (Split(500, 900, 2100), Split(10, 400, 2000), Split(1000, 1001, 1009)):
        cache.prune(0, s, inv)
        torch.cuda.synchronize()
        cos, sin = osp.rope_table(-s.gap, inv)
        nxt = []
        for layer, (k, v) in enumerate(cur):
            kb, vb, nn = osp.splice_growing(k, v, k.shape[1], s.a, s.c0, s.c, cos, sin, "bfloat16")
            gk, gv = cache.gather(layer)
            assert np.array_equal(bits(gk), kb[:, :nn].view(np.int16))
            assert np.array_equal(bits(gv), vb[:, :nn].view(np.int16))
            nxt.append((kb[:, :nn], vb[:, :nn]))
        cur = nxt
    assert cache.length() == 2009


@pytest.mark.parametrize("lens,P,dt", [([777], 64, torch.float16), ([3000, 17, 1, 640], 16, torch.float16),
                                       ([15, 4000], 48, torch.float16), ([1500, 33], 32, torch.bfloat16)])
def test_fused_paged_append_matches_append_then_decode(gpu, lens, P, dt):
    """reserve_step + decode_append against append (torch row writes) + decode on
    a twin cache: the pools end bit-identical and the outputs agree; both match
    the closed form. Two steps in a row, so the second attends the first's row."""
    layers, g = 2, 4
    print(f"case: fused paged append lens={lens} P={P} {dt}", flush=True)
    fused, host = filled(gpu, layers, lens, P, seed=61, dtype=dt)
    twin, _ = filled(gpu, layers, lens, P, seed=61, dtype=dt)
    gen = torch.Generator().manual_seed(62)
    B = len(lens)
    for step in range(2):
        kn = [torch.randn(B, 8, 128, generator=gen).to(dt) for _ in range(layers)]
        vn = [torch.randn(B, 8, 128, generator=gen).to(dt) for _ in range(layers)]
        qs = [torch.randn(B, 8, g, 128, generator=gen).to(dt) for _ in range(layers)]
        fused.reserve_step()
        outs = [fused.decode_append(layer, qs[layer].to(gpu), kn[layer].to(gpu), vn[layer].to(gpu), SCALE)
                for layer in range(layers)]
        for b in range(B):
            twin.append(b, [kn[layer][b].unsqueeze(1).to(gpu) for layer in range(layers)],
                        [vn[layer][b].unsqueeze(1).to(gpu) for layer in range(layers)])
        torch.cuda.synchronize()
        for layer in range(layers):
            want = twin.decode(layer, qs[layer].to(gpu), SCALE)
            torch.cuda.synchronize()
            # Same math in another order: the stored outputs may differ by one ulp of the result.
            diff = (outs[layer].float() - want.float()).abs() - (1e-3 + 2 * HALF_ULP[dt] * want.float().abs())
            assert diff.max().item() <= 0
            for b in range(B):
                host[b][layer] = (torch.cat([host[b][layer][0], kn[layer][b].unsqueeze(1)], dim=1),
                                  torch.cat([host[b][layer][1], vn[layer][b].unsqueeze(1)], dim=1))
                fk, fv = fused.gather(layer, b)
                tk, tv = twin.gather(layer, b)
                assert torch.equal(fk, tk) and torch.equal(fv, tv)
                assert torch.equal(fk.cpu(), host[b][layer][0])
                want64 = closed_form(qs[layer][b], *host[b][layer])
                excess = np.abs(outs[layer][b].float().cpu().numpy() - want64) - (TOL[dt] + HALF_ULP[dt] * np.abs(want64))
                assert excess.max() <= 0
    with pytest.raises(RuntimeError, match="reserve_step"):
        fused.decode_append(0, qs[0].to(gpu), kn[0].to(gpu), vn[0].to(gpu), SCALE)


@pytest.mark.parametrize("past", [0, 5])
def test_device_length_step_past_the_offset_rows_writes_nothing(gpu, past):
    """tc_decode_paged_append_attention_at with lens[b] at or past the offset table's rows
    (no slot holds position lens[b]): the pools stay unchanged, and the output is attention
    over the cached rows below lens[b] that the table holds plus the new token."""
    n, P = 100, 16
    cache, host = filled(gpu, 1, [n], P, seed=71)
    off, pitch = cache.device_offsets()
    assert pitch == n
    gen = torch.Generator().manual_seed(72)
    q = torch.randn(1, 8, 4, 128, generator=gen).half()
    kn = torch.randn(1, 8, 128, generator=gen).half()
    vn = torch.randn(1, 8, 128, generator=gen).half()
    before = (cache.k_pools[0].clone(), cache.v_pools[0].clone())
    lens = torch.tensor([n + past], dtype=torch.int32, device=gpu)
    print(f"case: device-length step at lens={n + past}, pitch={pitch}", flush=True)
    out = cache.decode_append_at(0, q.to(gpu), kn.to(gpu), vn.to(gpu), lens, SCALE)
    torch.cuda.synchronize()
    assert torch.equal(cache.k_pools[0], before[0]) and torch.equal(cache.v_pools[0], before[1])
    k = torch.cat([host[0][0][0], kn[0].unsqueeze(1)], dim=1)
    v = torch.cat([host[0][0][1], vn[0].unsqueeze(1)], dim=1)
    want = closed_form(q[0], k, v)
    assert np.abs(out[0].float().cpu().numpy() - want).max() <= TOL[torch.float16]


def test_decode_and_prune_refused_while_a_step_is_pending(gpu):
    """After reserve_step() the tile table holds each sequence's unwritten slot: decode() of a
    layer refuses until that layer has run decode_append, prune() until every layer has (or
    cancel_step() drops the slots)."""
    cache, host = filled(gpu, 2, [100, 40], 16, 71)
    g = torch.Generator(device=gpu)
    g.manual_seed(71)
    q = torch.randn((2, 8, 4, 128), generator=g, device=gpu).half()
    kn = torch.randn((2, 8, 128), generator=g, device=gpu).half()
    before = [cache.length(0), cache.length(1)]
    cache.reserve_step()
    assert [cache.length(0), cache.length(1)] == [101, 41]
    with pytest.raises(RuntimeError, match="incomplete"):
        cache.decode(0, q, SCALE)
    with pytest.raises(RuntimeError, match="incomplete"):
        cache.prune(0, Split(10, 20, 30), workloads.inv_freq())
    with pytest.raises(RuntimeError, match="incomplete"):
        cache.reserve_step()
    cache.cancel_step()
    assert [cache.length(0), cache.length(1)] == before
    out = cache.decode(0, q, SCALE)  # the step is gone: the old keys decode as before
    torch.cuda.synchronize()
    for b in range(2):
        k, v = host[b][0]
        want = closed_form(q[b:b + 1].cpu(), k[None], v[None])
        assert np.abs(out[b:b + 1].float().cpu().numpy() - want).max() <= TOL[torch.float16]
    cache.reserve_step()
    fused = cache.decode_append(0, q, kn, kn, SCALE)
    with pytest.raises(RuntimeError, match="incomplete"):
        cache.decode(1, q, SCALE)
    with pytest.raises(RuntimeError, match="incomplete"):
        cache.prune(0, Split(10, 20, 30), workloads.inv_freq())
    with pytest.raises(RuntimeError, match="incomplete"):
        cache.reserve_step()
    again = cache.decode(0, q, SCALE)  # layer 0's row is written: it reads the new token from its slot
    torch.cuda.synchronize()
    assert (again.float() - fused.float()).abs().max().item() <= TOL[torch.float16]
    cache.decode_append(1, q, kn, kn, SCALE)
    cache.decode(1, q, SCALE)  # the step is complete
    cache.prune(0, Split(10, 20, 30), workloads.inv_freq())
    assert cache.length(0) == 40


def test_write_step_then_decode_reads_the_new_rows(gpu):
    """The unfused step order: write_step() puts each layer's new row into its reserved slot
    with torch copies; decode() then attends it like any cached token."""
    cache, host = filled(gpu, 2, [50, 9], 16, 72)
    g = torch.Generator(device=gpu)
    g.manual_seed(72)
    q = torch.randn((2, 8, 4, 128), generator=g, device=gpu).half()
    kn = [torch.randn((2, 8, 128), generator=g, device=gpu).half() for _ in range(2)]
    vn = [torch.randn((2, 8, 128), generator=g, device=gpu).half() for _ in range(2)]
    cache.reserve_step()
    with pytest.raises(RuntimeError, match="no reserved slot"):
        cache.write_step(5, kn[0], vn[0])
    for layer in range(2):
        cache.write_step(layer, kn[layer], vn[layer])
    with pytest.raises(RuntimeError, match="no reserved slot"):
        cache.write_step(0, kn[0], vn[0])
    for layer in range(2):
        out = cache.decode(layer, q, SCALE)
        torch.cuda.synchronize()
        for b in range(2):
            k, v = host[b][layer]
            k = torch.cat((k, kn[layer][b].cpu()[:, None]), 1)
            v = torch.cat((v, vn[layer][b].cpu()[:, None]), 1)
            want = closed_form(q[b:b + 1].cpu(), k[None], v[None])
            assert np.abs(out[b:b + 1].float().cpu().numpy() - want).max() <= TOL[torch.float16]


def test_cache_made_on_the_current_device_takes_its_tensors(gpu):
    """PagedKV(device="cuda") names the current device; it records the pools' own device, so
    queries on that device (with its index) are accepted and decoded."""
    cache = PagedKV(1, 8, 8, 16, device="cuda")
    assert cache.device.index == torch.cuda.current_device()
    k = torch.randn(8, 40, 128, generator=torch.Generator().manual_seed(70)).half()
    v = torch.randn(8, 40, 128, generator=torch.Generator().manual_seed(71)).half()
    dev = torch.device("cuda", torch.cuda.current_device())
    cache.append(0, [k.to(dev)], [v.to(dev)])
    q = torch.randn(1, 8, 4, 128, generator=torch.Generator().manual_seed(72)).half()
    out = cache.decode(0, q.to(dev), 128 ** -0.5)
    torch.cuda.synchronize()
    want = od.attention_f64(q.float().numpy(), k.float().numpy()[None], v.float().numpy()[None], 128 ** -0.5)
    assert np.abs(out.float().cpu().numpy() - want).max() <= 2e-3
