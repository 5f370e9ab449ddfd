"""Seeded random sweeps of the HIP paths against the oracle: shapes, lengths,
group sizes, element types, split lengths and masks drawn per case, so the
parity tests reach combinations the hand-picked cases do not.

- Decode (tc_decode_attention through decode_attention_batched): batches with
  and without per-sequence lengths (empty sequences included), g in 1..8,
  fixed or tuned split lengths, against the float64 closed form
  (threadcut/flash_decode.py:57-69): max-abs 2e-3 fp16; bf16 4e-3 plus its
  half-ulp of the value (2^-8 |x|), since a sequence of a few keys gives
  outputs of 2 and more, where the bf16 rounding of the exact result alone
  exceeds 4e-3.
- Splice (tc_splice_rope through kv.splice): random (a, c0, c) on random
  capacities, overlapping and disjoint, against the oracle's restatement of
  threadcut/kv.py:83-92: bit-exact.
- Prefill (tc_prefill_attention): random chunk shapes with no mask, is_causal,
  a causal chunk mask or a random mask, and forced key splits, against the
  float64 closed form of attention.py:43-46: 2e-3 fp16, 1.6e-2 bf16.
- The paged cache: random page sizes, appends and prunes; pages bit-exact
  against the contiguous splice of the same sequence, decode and prefill
  through the pools against the float64 closed form.
"""
import random

import numpy as np
import pytest
import torch

from oracle import decode as od
from oracle import prefill as opf
from oracle import splice as osp
from threadcut_amd import flash_decode, kv, prefill, workloads
from threadcut_amd.match import Split

pytestmark = pytest.mark.gpu

D = 128
DECODE_TOL = {torch.float16: 2e-3, torch.bfloat16: 4e-3}
DECODE_REL = {torch.float16: 0.0, torch.bfloat16: 2.0 ** -8}  # bf16: the half-ulp of the output value


def decode_excess(out, want, dtype):
    """Largest amount by which |out - want| exceeds the decode bound (<= 0 passes)."""
    return float((np.abs(out - want) - (DECODE_TOL[dtype] + DECODE_REL[dtype] * np.abs(want))).max())
PREFILL_TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


def decode_case(seed):
    r = random.Random(seed)
    b = r.choice([1, 1, 2, 3, 5])
    hkv = r.choice([1, 2, 4, 8])
    g = r.choice([1, 2, 3, 4, 5, 8])
    n = r.choice([1, 17, 300, 1536, 4097, r.randint(1, 16000)])
    dtype = r.choice([torch.float16, torch.bfloat16])
    split = r.choice([None, None, 64 * r.randint(1, 64)])
    ragged = b > 1 and r.random() < 0.6
    lens = torch.tensor([r.choice([0, 1, n, r.randint(0, n)]) for _ in range(b)], dtype=torch.int32) \
        if ragged else None
    return b, hkv, g, n, dtype, split, lens


# Seed 237 (bf16, a sequence of 3 keys) gives outputs above 2, where bf16 rounds in steps of 2^-6.
@pytest.mark.parametrize("seed", [*range(120), 237])
def test_random_decode(gpu, seed):
    b, hkv, g, n, dtype, split, lens = decode_case(seed)
    print(f"case: decode seed={seed} B={b} Hkv={hkv} g={g} n={n} {dtype} split={split} "
          f"lens={None if lens is None else lens.tolist()}", flush=True)
    gen = torch.Generator().manual_seed(1000 + seed)
    q = torch.randn(b, hkv, g, D, generator=gen).to(dtype)
    k = torch.randn(b, hkv, n, D, generator=gen).to(dtype)
    v = torch.randn(b, hkv, n, D, generator=gen).to(dtype)
    scale = D ** -0.5
    out = flash_decode.decode_attention_batched(q.to(gpu), k.to(gpu), v.to(gpu), scale,
                                                lens=None if lens is None else lens.to(gpu), split=split)
    torch.cuda.synchronize()
    qn, kn, vn = q.float().numpy(), k.float().numpy(), v.float().numpy()
    want = od.attention_f64(qn, kn, vn, scale) if lens is None else od.decode_ragged(qn, kn, vn, lens.numpy(), scale)
    assert decode_excess(out.float().cpu().numpy(), want, dtype) <= 0


class _Cache:
    def __init__(self, layers):
        self.layers = layers


@pytest.mark.parametrize("seed", range(80))
def test_random_splice(gpu, seed, monkeypatch):
    def no_torch(*args, **kwargs):
        raise AssertionError("a GPU splice reached the torch op sequence instead of the HIP kernel")

    for name in ("_splice_layer_torch", "_shift_keys_torch", "_splice_index_select_torch"):
        monkeypatch.setattr(kv, name, no_torch)
    r = random.Random(seed)
    layers, batch, heads = r.randint(1, 3), r.choice([1, 1, 2]), r.choice([1, 2, 8])
    n = r.randint(2, 6000)
    a = r.randint(0, n - 1)
    c0 = r.choice([a, a + 1, a + r.randint(1, 47), a + r.randint(48, 700), r.randint(a, n)])
    c0 = min(c0, n)
    c = r.randint(0, n - c0)
    dtype = r.choice([torch.float16, torch.bfloat16])
    s = Split(a, c0, c)
    print(f"case: splice seed={seed} L={layers} B={batch} H={heads} n={n} {s} {dtype}", flush=True)
    ks, vs = workloads.layer_caches(2000 + seed, layers, n, kv_heads=heads, batch=batch, dtype=dtype)
    inv = workloads.inv_freq(1e6)
    cache_layers = []
    for k, v in zip(ks, vs):
        layer = kv.GrowingLayer()
        layer.update(k.to(gpu), v.to(gpu))
        cache_layers.append(layer)
    kv.splice(_Cache(cache_layers), s, inv)
    torch.cuda.synchronize()
    name = "float16" if dtype == torch.float16 else "bfloat16"
    cos, sin = osp.rope_table(-s.gap, inv)
    for i, layer in enumerate(cache_layers):
        kn = ks[i].view(torch.int16).numpy().view(np.uint16) if name == "bfloat16" else ks[i].numpy()
        vn = vs[i].view(torch.int16).numpy().view(np.uint16) if name == "bfloat16" else vs[i].numpy()
        kb, vb, nn = osp.splice_growing(kn, vn, n, s.a, s.c0, s.c, cos, sin, name)
        assert layer.n == nn == s.a + s.c
        got_k = layer.kbuf[..., :n, :].cpu().view(torch.int16).numpy()
        got_v = layer.vbuf[..., :n, :].cpu().view(torch.int16).numpy()
        assert np.array_equal(got_k, np.asarray(kb).view(np.int16)), f"K layer {i}"
        assert np.array_equal(got_v, np.asarray(vb).view(np.int16)), f"V layer {i}"


@pytest.mark.parametrize("seed", range(50))
def test_random_prefill(gpu, seed):
    r = random.Random(seed)
    b = r.choice([1, 1, 2])
    hkv = r.choice([1, 2, 4, 8])
    g = r.choice([1, 2, 4, 8])
    mode = r.choice(["none", "causal", "chunk", "random"])
    q_len = r.randint(1, 400)
    n = q_len if mode == "causal" else q_len + r.randint(0, 1600)
    dtype = r.choice([torch.float16, torch.bfloat16])
    splits = r.choice([None, None, r.randint(1, 8)])
    print(f"case: prefill seed={seed} B={b} Hkv={hkv} g={g} q={q_len} n={n} {mode} {dtype} splits={splits}",
          flush=True)
    q, k, v = workloads.prefill_inputs(3000 + seed, batch=b, q_len=q_len, n=n, q_heads=hkv * g, kv_heads=hkv,
                                       dtype=dtype)
    mask = None
    if mode == "chunk":
        mask = workloads.causal_mask(q_len, n)
    elif mode == "random":
        gen = torch.Generator().manual_seed(4000 + seed)
        mask = torch.rand((r.choice([1, b]), 1, q_len, n), generator=gen) < r.choice([0.05, 0.5, 0.95])
    scale = D ** -0.5
    out = prefill.prefill_attention(q.to(gpu), k.to(gpu), v.to(gpu), None if mask is None else mask.to(gpu),
                                    scale, mode == "causal", splits=splits)
    torch.cuda.synchronize()
    want = opf.prefill_f64(q.float().numpy(), k.float().numpy(), v.float().numpy(), scale,
                           mask=None if mask is None else mask.numpy(), causal=mode == "causal")
    assert np.abs(out.float().cpu().numpy() - want).max() <= PREFILL_TOL[dtype]


@pytest.mark.parametrize("seed", range(40))
def test_random_paged(gpu, seed):
    """The paged cache: random page size, appends in random chunks from a shuffled free
    list, zero to two random prunes; the pages against the contiguous splice of the same
    sequence (bit-exact), then decode and prefill against the float64 closed form on the
    gathered keys."""
    from threadcut_amd.paged import PagedKV

    r = random.Random(seed)
    P = r.choice([16, 32, 48, 64, 128])
    hkv, g = r.choice([(8, 4), (4, 8), (2, 2), (8, 1)])
    dtype = r.choice([torch.float16, torch.bfloat16])
    n = r.randint(1, 5000)
    name = "float16" if dtype == torch.float16 else "bfloat16"
    pages = -(-n // P) * 2 + 8
    cache = PagedKV(1, hkv, pages, P, dtype=dtype, device=gpu)
    r.shuffle(cache.table.free)
    gen = torch.Generator().manual_seed(5000 + seed)
    k = torch.randn(hkv, n, D, generator=gen).to(dtype)
    v = torch.randn(hkv, n, D, generator=gen).to(dtype)
    done = 0
    while done < n:
        m = min(n - done, r.choice([1, 7, 16, 64, 300, 1500]))
        cache.append(0, [k[:, done:done + m].to(gpu)], [v[:, done:done + m].to(gpu)])
        done += m
    inv = workloads.inv_freq(1e6)
    kn = (k.view(torch.int16).numpy().view(np.uint16) if name == "bfloat16" else k.numpy())[None]
    vn = (v.view(torch.int16).numpy().view(np.uint16) if name == "bfloat16" else v.numpy())[None]
    splits = []
    for _ in range(r.choice([0, 1, 2])):
        cur = cache.length()
        if cur < 2:
            break
        a = r.randint(0, cur - 1)
        c0 = r.randint(a, cur)
        c = r.randint(0, cur - c0)
        s = Split(a, c0, c)
        splits.append(s)
        cache.prune(0, s, inv)
        cos, sin = osp.rope_table(-s.gap, inv)
        kn, vn, nn = osp.splice_growing(kn, vn, cur, s.a, s.c0, s.c, cos, sin, name)
        kn, vn = kn[..., :nn, :], vn[..., :nn, :]
    print(f"case: paged seed={seed} P={P} Hkv={hkv} g={g} n={n} {dtype} prunes={splits}", flush=True)
    gk, gv = cache.gather(0)
    torch.cuda.synchronize()
    assert gk.shape[1] == kn.shape[-2] == cache.length()
    assert np.array_equal(gk.cpu().view(torch.int16).numpy(), np.asarray(kn[0]).view(np.int16))
    assert np.array_equal(gv.cpu().view(torch.int16).numpy(), np.asarray(vn[0]).view(np.int16))
    keys, vals = gk.cpu().float().numpy()[None], gv.cpu().float().numpy()[None]
    q = torch.randn(1, hkv, g, D, generator=gen).to(dtype)
    out = cache.decode(0, q.to(gpu), D ** -0.5)
    torch.cuda.synchronize()
    want = od.attention_f64(q.float().numpy(), keys, vals, D ** -0.5)
    assert decode_excess(out.float().cpu().numpy(), want, dtype) <= 0
    nq = r.randint(1, min(cache.length(), 200)) if cache.length() else 0
    if nq:
        qp = torch.randn(1, nq, hkv * g, D, generator=gen).to(dtype).transpose(1, 2)
        outp = cache.prefill(0, qp.to(gpu), D ** -0.5, causal=False)
        torch.cuda.synchronize()
        wantp = opf.prefill_f64(qp.float().numpy(), keys, vals, D ** -0.5)
        assert np.abs(outp.float().cpu().numpy() - wantp).max() <= PREFILL_TOL[dtype]
