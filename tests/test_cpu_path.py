"""Host tensors through the drop-in: the reference's own CPU path, on the CPU.

The reference runs decode as SDPA with the query heads folded
(threadcut/attention.py:40-42) and shift_keys / splice / GrowingLayer.splice
as torch ops (threadcut/kv.py:20-41, 83-92) for tensors its GPU kernel does
not take; its CPU CI (tests/test_core.py) pins them with T1, T2 and the
growing-vs-copy splice on a tiny fp32 Qwen3 (head_dim 16). The same checks
run here through threadcut_amd, plus bit-level comparisons with the oracle's
restatement of the reference's op sequences.
"""
import numpy as np
import pytest
import torch
from transformers import AutoModelForCausalLM, DynamicCache, Qwen3Config
from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding

from oracle import decode as od
from oracle import splice as osp
from threadcut_amd import attention, kv, workloads
from threadcut_amd.match import Split, split


def rope_at(rot, x, p):
    cos, sin = rot(x, torch.full((1, x.shape[2]), p, dtype=torch.long))
    return x * cos[:, None].float() + kv.rotate_half(x) * sin[:, None].float()


@pytest.mark.parametrize("head_dim,theta", [(16, 1e4), (128, 1e6)])
def test_T1_shift_is_rotation_composition(head_dim, theta):
    """tests/test_core.py:67-74 through threadcut_amd.kv.shift_keys on host fp32 keys:
    shift(rope(k, 900), -350) == rope(k, 550) with transformers' own rotary embedding."""
    rot = Qwen3RotaryEmbedding(Qwen3Config(head_dim=head_dim, rope_theta=theta, max_position_embeddings=4096))
    k = torch.randn(1, 2, 5, head_dim, generator=torch.Generator().manual_seed(0))
    shifted = kv.shift_keys(rope_at(rot, k, 900), -350, rot.inv_freq)
    assert shifted.dtype == torch.float32 and shifted.device.type == "cpu"
    assert torch.allclose(shifted, rope_at(rot, k, 550), atol=1e-4)


def test_growing_layer_splice_matches_copy_splice():
    """tests/test_core.py:104-121 through threadcut_amd: the in-place GrowingLayer splice equals the
    index_select splice of a plain DynamicCache, for an overlapping move and an empty suffix, and
    appending after a splice keeps working."""
    torch.manual_seed(0)
    k, v = torch.randn(1, 2, 40, 16), torch.randn(1, 2, 40, 16)
    inv_freq = 1.0 / (10000 ** (torch.arange(0, 16, 2).float() / 16))
    for s in (Split(10, 17, 20), Split(12, 12, 0)):
        grown = kv.GrowingLayer()
        grown.update(k, v)
        grown.splice(s, inv_freq)
        ref = DynamicCache(config=Qwen3Config(num_hidden_layers=1))
        ref.layers[0].update(k, v)
        kv.splice(ref, s, inv_freq)
        assert torch.allclose(grown.keys, ref.layers[0].keys) and torch.allclose(grown.values, ref.layers[0].values)
        assert grown.keys.shape[-2] == s.a + s.c
        grown.update(k[:, :, :3], v[:, :, :3])
        assert grown.get_seq_length() == s.a + s.c + 3


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_host_splice_is_the_reference_op_sequence(dtype):
    """fp16/bf16 host buffers at the Qwen3 head shape: GrowingLayer splice (via kv.splice) and
    shift_keys are bit-identical to the oracle's restatement of threadcut/kv.py:20-25, 83-92."""
    tdt = getattr(torch, dtype)
    s = Split(10, 17, 20)
    inv = workloads.inv_freq(1e6)
    ks, vs = workloads.layer_caches(1, 2, 64, dtype=tdt)
    cache = kv.new_cache(Qwen3Config(num_hidden_layers=2, head_dim=128))
    for layer, kk, vv in zip(cache.layers, ks, vs):
        layer.update(kk, vv)
    kv.splice(cache, s, inv)
    cos, sin = osp.rope_table(-s.gap, inv)
    for layer, kk, vv in zip(cache.layers, ks, vs):
        kb, vb, n = osp.splice_growing(od.to_dtype_bits(kk.float().numpy(), dtype), od.to_dtype_bits(
            vv.float().numpy(), dtype), 64, s.a, s.c0, s.c, cos, sin, dtype=dtype)
        assert n == layer.n == 30
        got_k = od.to_dtype_bits(layer.kbuf[:, :, :64].float().numpy(), dtype)
        got_v = od.to_dtype_bits(layer.vbuf[:, :, :64].float().numpy(), dtype)
        assert np.array_equal(got_k.view(np.uint16), np.asarray(kb).view(np.uint16))
        assert np.array_equal(got_v.view(np.uint16), np.asarray(vb).view(np.uint16))
    keys = ks[0][:, :, 5:25]
    got = kv.shift_keys(keys, -300, inv)
    c3, s3 = osp.rope_table(-300, inv)
    want = osp.shift_keys(od.to_dtype_bits(keys.float().numpy(), dtype), c3, s3, dtype)
    assert np.array_equal(od.to_dtype_bits(got.float().numpy(), dtype).view(np.uint16),
                          np.asarray(want).view(np.uint16))


def test_host_splice_rejects_a_suffix_past_the_cache():
    layer = kv.GrowingLayer()
    k = torch.randn(1, 2, 20, 16)
    layer.update(k, k)
    with pytest.raises(ValueError):
        layer.splice(Split(2, 5, 30), torch.ones(8))


@pytest.mark.parametrize("b,hq,hkv,n", [(1, 4, 2, 33), (2, 32, 8, 300), (1, 16, 1, 7)])
def test_host_decode_is_folded_sdpa(b, hq, hkv, n):
    """threadcut/attention.py:40-42 on host fp32 tensors: equal to the oracle's folded SDPA and
    within fp32 rounding of the float64 closed form; output [b, 1, hq, d] contiguous."""
    d = 16 if hq == 4 else 64
    g = torch.Generator().manual_seed(n)
    q = torch.randn(b, hq, 1, d, generator=g)
    k = torch.randn(b, hkv, n, d, generator=g)
    v = torch.randn(b, hkv, n, d, generator=g)
    out, none = attention.attention(None, q, k, v, None, scaling=d ** -0.5)
    assert none is None and out.shape == (b, 1, hq, d) and out.is_contiguous()
    ref = od.folded_sdpa(q, k, v, d ** -0.5).transpose(1, 2)
    assert torch.equal(out, ref.contiguous())
    f64 = od.attention_f64(q.numpy().reshape(b, hkv, hq // hkv, d), k.numpy(), v.numpy(), d ** -0.5)
    assert np.abs(out.numpy().reshape(b, hkv, hq // hkv, d) - f64).max() < 1e-5


def tiny_model():
    """The reference's tiny CPU model (tests/test_core.py:16-22) with the "threadcut" attention."""
    torch.manual_seed(0)
    cfg = Qwen3Config(vocab_size=512, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=16, max_position_embeddings=4096)
    return AutoModelForCausalLM.from_config(cfg, dtype=torch.float32, attn_implementation=attention.NAME).eval()


def rand_ids(n, seed, vocab=500):
    return torch.randint(10, vocab, (n,), generator=torch.Generator().manual_seed(seed)).tolist()


def kv_alone(model, ids, start):
    cache = DynamicCache(config=model.config)
    pos = torch.arange(start, start + len(ids))[None]
    model(input_ids=torch.tensor([ids]), position_ids=pos, past_key_values=cache, use_cache=True)
    return cache


def forward_chunks(model, ids, cache, chunk=7):
    logits = None
    for i in range(0, len(ids), chunk):
        logits = model(input_ids=torch.tensor([ids[i:i + chunk]]), past_key_values=cache, use_cache=True,
                       logits_to_keep=1).logits[0, -1]
    return logits


@pytest.fixture
def decode_calls(monkeypatch):
    """Counts the attention calls that take the decode branch (one query token, no mask)."""
    calls = []
    gate = attention.decode_supports

    def counted(query, key, value):
        calls.append(tuple(query.shape))
        return gate(query, key, value)

    monkeypatch.setattr(attention, "decode_supports", counted)
    return calls


@pytest.mark.parametrize("growing", [False, True, "slab"])
@torch.no_grad()
def test_T2_splice_matches_fresh_compute(growing, decode_calls):
    """tests/test_core.py:77-90 with the "threadcut" attention on the CPU: a cache A·B·C (C placed
    after B without seeing it) spliced to A·C and continued with D gives the logits of A, then C
    placed after A, then D. The suffix is found with match.split (min_suffix 4) and the cache is
    spliced with kv.splice, as engine.py:51-59 does; D runs in chunks of 7 and token by token."""
    m = tiny_model()
    inv = m.model.rotary_emb.inv_freq
    A, B, C, D = rand_ids(9, 1), rand_ids(13, 2), rand_ids(11, 3), rand_ids(5, 4)
    for chunk in (7, 1):
        ref = kv_alone(m, A, 0)
        for lr, lc in zip(ref.layers, kv_alone(m, C, len(A)).layers):
            lr.keys, lr.values = torch.cat((lr.keys, lc.keys), 2), torch.cat((lr.values, lc.values), 2)
        ref_logits = forward_chunks(m, D, ref, chunk)
        parts = [kv_alone(m, A, 0), kv_alone(m, B, len(A)), kv_alone(m, C, len(A) + len(B))]
        cache = kv.new_cache(m.config, slab=growing == "slab") if growing else DynamicCache(config=m.config)
        for i, layer in enumerate(cache.layers):
            layer.update(torch.cat([p.layers[i].keys for p in parts], 2),
                         torch.cat([p.layers[i].values for p in parts], 2))
        s = split(A + B + C, A + C + D, 4)
        assert (s.a, s.c0, s.c) == (9, 22, 11)
        kv.splice(cache, s, inv)
        assert cache.get_seq_length() == 20
        logits = forward_chunks(m, (A + C + D)[s.a + s.c:], cache, chunk)
        assert torch.allclose(logits, ref_logits, atol=1e-4, rtol=0), (chunk, (logits - ref_logits).abs().max())
    assert len(decode_calls) >= 2 * len(D)  # the token-by-token pass ran the decode branch in every layer


@torch.no_grad()
def test_decode_steps_match_stock_sdpa(decode_calls):
    """Token-by-token decode of the tiny model with the "threadcut" attention over a GrowingLayer
    cache equals transformers' stock SDPA attention over its own cache."""
    m = tiny_model()
    prompt, steps = rand_ids(17, 5), rand_ids(6, 6)
    c1 = kv.new_cache(m.config)
    c2 = DynamicCache(config=m.config)
    m(input_ids=torch.tensor([prompt]), past_key_values=c1, use_cache=True)
    m.set_attn_implementation("sdpa")
    m(input_ids=torch.tensor([prompt]), past_key_values=c2, use_cache=True)
    for t in steps:
        m.set_attn_implementation(attention.NAME)
        a = m(input_ids=torch.tensor([[t]]), past_key_values=c1, use_cache=True).logits[0, -1]
        m.set_attn_implementation("sdpa")
        b = m(input_ids=torch.tensor([[t]]), past_key_values=c2, use_cache=True).logits[0, -1]
        assert torch.allclose(a, b, atol=1e-5, rtol=0)
    assert len(decode_calls) == 2 * len(steps)  # 2 layers per step, all through the decode branch


def test_slab_layers_share_one_allocation_through_growth():
    """new_cache(slab=True) on the host: the layers' buffers are views of one [L, 2, B, Hkv, cap, D]
    tensor before and after a growth, and each layer keeps its own tokens."""
    cfg = Qwen3Config(num_hidden_layers=3, head_dim=16, num_key_value_heads=2)
    cache = kv.new_cache(cfg, slab=True)
    g = torch.Generator().manual_seed(5)
    rows = [(torch.randn(1, 2, 2000, 16, generator=g), torch.randn(1, 2, 2000, 16, generator=g)) for _ in range(3)]
    for layer, (k, v) in zip(cache.layers, rows):
        layer.update(k, v)
    t = cache.layers[0].slab.tensor
    assert t.shape == (3, 2, 1, 2, 2048, 16)
    for layer, (k, v) in zip(cache.layers, rows):
        layer.update(k[:, :, :100], v[:, :, :100])  # past 2048: grows once, for every layer
    t2 = cache.layers[0].slab.tensor
    assert t2.shape[-2] == 4096 and t2.untyped_storage().data_ptr() != t.untyped_storage().data_ptr()
    for i, (layer, (k, v)) in enumerate(zip(cache.layers, rows)):
        assert layer.kbuf.untyped_storage().data_ptr() == t2.untyped_storage().data_ptr()
        assert layer.kbuf.data_ptr() == t2[i, 0].data_ptr() and layer.vbuf.data_ptr() == t2[i, 1].data_ptr()
        assert layer.keys.shape == (1, 2, 2100, 16)
        assert torch.equal(layer.keys, torch.cat((k, k[:, :, :100]), 2))
        assert torch.equal(layer.values, torch.cat((v, v[:, :, :100]), 2))


def test_decode_graph_refuses_a_model_on_another_attention():
    """The captured decode step leaves each layer's new K/V row to the "threadcut" decode kernel;
    a model switched to another attention would attend over an unwritten row, so DecodeGraph
    refuses it before it touches the cache or a device."""
    from threadcut_amd.graph import DecodeGraph

    m = tiny_model()
    m.set_attn_implementation("sdpa")
    with pytest.raises(ValueError, match="set_attn_implementation"):
        DecodeGraph(m, kv.new_cache(m.config), max_new_tokens=4)
