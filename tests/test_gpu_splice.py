"""Splice / RoPE-shift parity on the GPU: HIP kernels vs the CPU oracle, bit for bit.

V moves and index remaps must be bit-exact; shifted K is bit-exact too (the
kernel follows the reference's fp32 op order with the same host cos/sin
table), which implies the 2e-3 bound.
"""
import numpy as np
import pytest
import torch
from transformers import DynamicCache, Qwen3Config

from oracle import splice as osp
from threadcut_amd import kv, workloads
from threadcut_amd.match import Split

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def kernels_only(monkeypatch):
    """Every splice here runs on GPU buffers, so it must take the HIP kernels: the reference's
    torch op sequences (what host buffers run) raise if anything routes to them. The torch
    ops give the oracle's bits too, so without this guard a routing mistake would pass."""
    def no_torch(*args, **kwargs):
        raise AssertionError("a GPU splice reached the torch op sequence instead of the HIP kernel")

    for name in ("_splice_layer_torch", "_shift_keys_torch", "_splice_index_select_torch"):
        monkeypatch.setattr(kv, name, no_torch)


def bits(t):
    if isinstance(t, torch.Tensor):
        t = t.detach().cpu()
        return t.view(torch.int16).numpy()
    return np.asarray(t).view(np.int16)


class Cache:
    def __init__(self, layers):
        self.layers = layers


def growing_cache(ks, vs, dev, extra=0):
    layers = []
    for k, v in zip(ks, vs):
        layer = kv.GrowingLayer()
        layer.update(k.to(dev), v.to(dev))
        if extra:
            layer._reserve(layer.n + extra, layer.kbuf)
        layers.append(layer)
    return Cache(layers)


def oracle_splice(k, v, s, inv, dtype="float16"):
    cos, sin = osp.rope_table(-s.gap, inv)
    kn = k.numpy() if dtype == "float16" else k.view(torch.int16).numpy().view(np.uint16)
    vn = v.numpy() if dtype == "float16" else v.view(torch.int16).numpy().view(np.uint16)
    return osp.splice_growing(kn, vn, k.shape[2], s.a, s.c0, s.c, cos, sin, dtype)


def test_full_splice_36_layers(gpu):
    """36 x [1, 8, 14336, 128] fp16 (seed 1), Split(2048, 8668, 5668), theta 1e6."""
    s = workloads.SPLICE_SPLIT
    ks, vs = workloads.layer_caches(1, 36, workloads.SPLICE_TOKENS)
    inv = workloads.inv_freq(1e6)
    cache = growing_cache(ks, vs, gpu)
    print("case: 36-layer splice", flush=True)
    kv.splice(cache, s, inv)
    torch.cuda.synchronize()
    for i, layer in enumerate(cache.layers):
        kb, vb, n = oracle_splice(ks[i], vs[i], s, inv)
        assert layer.n == n == s.a + s.c
        assert layer.keys.shape[2] == n
        assert np.array_equal(bits(layer.kbuf[:, :, :kb.shape[2]]), bits(kb)), f"K layer {i}"
        assert np.array_equal(bits(layer.vbuf[:, :, :vb.shape[2]]), bits(vb)), f"V layer {i}"


@pytest.mark.parametrize("s", [Split(10, 17, 20), Split(12, 12, 0), Split(0, 1, 4000), Split(100, 200, 3000),
                               Split(100, 229, 3000), Split(5, 4000, 1001), Split(3, 9, 4992), Split(0, 0, 50),
                               Split(100, 700, 4000), Split(0, 512, 4400), Split(7, 518, 511),
                               Split(0, 1000, 4001), Split(0, 32, 4000), Split(2, 34, 33), Split(3, 103, 4001),
                               Split(0, 511, 4490), Split(50, 300, 4701), Split(1, 32, 4000), Split(0, 47, 4000),
                               Split(1, 49, 4000), Split(0, 500, 4000), Split(0, 500, 4001), Split(9, 609, 4392),
                               Split(5, 52, 300), Split(0, 40, 290), Split(7, 8, 257), Split(3, 20, 1111),
                               Split(0, 45, 4000), Split(2, 48, 1000)])
def test_overlapping_and_edge_splits(gpu, s):
    n = 5001
    ks, vs = workloads.layer_caches(21, 3, n)
    inv = workloads.inv_freq(1e6)
    cache = growing_cache(ks, vs, gpu, extra=100)
    print(f"case: {s}", flush=True)
    kv.splice(cache, s, inv)
    torch.cuda.synchronize()
    for i, layer in enumerate(cache.layers):
        kb, vb, nn = oracle_splice(ks[i], vs[i], s, inv)
        assert layer.n == nn
        cap_n = ks[i].shape[2]
        assert np.array_equal(bits(layer.kbuf[:, :, :cap_n]), bits(kb))
        assert np.array_equal(bits(layer.vbuf[:, :, :cap_n]), bits(vb))


def test_reference_known_answer_growing_vs_copy(gpu):
    """The reference's test_growing_layer_splice_matches_copy_splice at head_dim 128."""
    g = torch.Generator().manual_seed(0)
    k = torch.randn(1, 2, 40, 128, generator=g).half().to(gpu)
    v = torch.randn(1, 2, 40, 128, generator=g).half().to(gpu)
    inv = 1.0 / (10000 ** (torch.arange(0, 128, 2).float() / 128))
    for s in (Split(10, 17, 20), Split(12, 12, 0)):
        grown = kv.GrowingLayer()
        grown.update(k, v)
        grown.splice(s, inv)
        ref = DynamicCache(config=Qwen3Config(num_hidden_layers=1))
        ref.layers[0].update(k, v)
        kv.splice(ref, s, inv)
        torch.cuda.synchronize()
        assert torch.equal(grown.keys, ref.layers[0].keys) and torch.equal(grown.values, ref.layers[0].values)
        grown.update(k[:, :, :3], v[:, :, :3])
        assert grown.get_seq_length() == s.a + s.c + 3
        assert torch.equal(grown.keys[:, :, -3:], k[:, :, :3])


def test_copy_splice_matches_oracle(gpu):
    """index_select branch (plain DynamicLayer caches) vs the oracle's splice_copy."""
    ks, vs = workloads.layer_caches(22, 4, 3000)
    inv = workloads.inv_freq(1e6)
    cache = DynamicCache(config=Qwen3Config(num_hidden_layers=4))
    for layer, k, v in zip(cache.layers, ks, vs):
        layer.update(k.to(gpu), v.to(gpu))
    s = Split(700, 1500, 1200)
    kv.splice(cache, s, inv)
    torch.cuda.synchronize()
    cos, sin = osp.rope_table(-s.gap, inv)
    for layer, k, v in zip(cache.layers, ks, vs):
        rk, rv = osp.splice_copy(k.numpy(), v.numpy(), s.a, s.c0, s.c, cos, sin)
        assert layer.keys.shape[2] == s.a + s.c
        assert np.array_equal(bits(layer.keys), bits(rk))
        assert np.array_equal(bits(layer.values), bits(rv))


@pytest.mark.parametrize("s", [Split(0, 5, 0), Split(0, 0, 0), Split(0, 300, 0)])
def test_copy_splice_keeping_nothing(gpu, s):
    """A split that keeps no token empties a plain DynamicLayer cache, as the reference's
    index_select does (threadcut/kv.py:34-41); appends continue from position 0."""
    ks, vs = workloads.layer_caches(24, 2, 300)
    cache = DynamicCache(config=Qwen3Config(num_hidden_layers=2))
    for layer, k, v in zip(cache.layers, ks, vs):
        layer.update(k.to(gpu), v.to(gpu))
    kv.splice(cache, s, workloads.inv_freq(1e6))
    for layer, k, v in zip(cache.layers, ks, vs):
        assert layer.keys.shape == (1, 8, 0, 128) and layer.values.shape == (1, 8, 0, 128)
        layer.update(k[:, :, :3].to(gpu), v[:, :, :3].to(gpu))
        assert torch.equal(layer.keys.cpu(), k[:, :, :3]) and torch.equal(layer.values.cpu(), v[:, :, :3])


def test_shift_keys_matches_oracle_and_reference_ops(gpu):
    g = torch.Generator().manual_seed(23)
    kbuf = torch.randn(2, 8, 600, 128, generator=g).half()
    view = kbuf[:, :, 37:537]  # a non-contiguous slice, as kbuf[..., c0:c0+c, :]
    inv = workloads.inv_freq(1e6)
    out = kv.shift_keys(view.to(gpu), -350, inv)
    torch.cuda.synchronize()
    cos, sin = osp.rope_table(-350, inv)
    assert np.array_equal(bits(out), bits(osp.shift_keys(view.numpy(), cos, sin)))
    # The reference's op sequence, threadcut/kv.py:20-25, on the CPU.
    kf = view.float()
    angle = -350 * inv.float()
    emb = torch.cat((angle, angle))
    ref = (kf * emb.cos() + kv.rotate_half(kf) * emb.sin()).to(torch.float16)
    assert torch.equal(out.cpu(), ref)


def test_shift_is_rotation_composition_fp16(gpu):
    """T1 in fp16: shift(rope(k, 900), -350) ≈ rope(k, 550), RoPE from transformers."""
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding

    cfg = Qwen3Config(head_dim=128, rope_theta=1e6, max_position_embeddings=4096)
    rot = Qwen3RotaryEmbedding(cfg)
    k = torch.randn(1, 2, 5, 128, generator=torch.Generator().manual_seed(24))

    def rope_at(x, p):
        cos, sin = rot(x, torch.full((1, x.shape[2]), p, dtype=torch.long))
        return x * cos[:, None].float() + kv.rotate_half(x) * sin[:, None].float()

    shifted = kv.shift_keys(rope_at(k, 900).half().to(gpu), -350, rot.inv_freq).float().cpu()
    want = rope_at(k, 550)
    # fp16 input and output rounding: two half-ulps of values below 8.
    assert (shifted - want).abs().max().item() <= 2 * 2 ** -8


@pytest.mark.parametrize("s", [Split(100, 900, 1000), Split(100, 170, 1830), Split(4, 20, 1900)])
def test_bf16_splice(gpu, s):
    ks, vs = workloads.layer_caches(25, 2, 2000, dtype=torch.bfloat16)
    inv = workloads.inv_freq(1e6)
    cache = growing_cache(ks, vs, gpu)
    print(f"case: {s}", flush=True)
    kv.splice(cache, s, inv)
    torch.cuda.synchronize()
    for i, layer in enumerate(cache.layers):
        kb, vb, _ = oracle_splice(ks[i], vs[i], s, inv, dtype="bfloat16")
        assert np.array_equal(bits(layer.kbuf[:, :, :2000]), bits(kb))
        assert np.array_equal(bits(layer.vbuf[:, :, :2000]), bits(vb))
