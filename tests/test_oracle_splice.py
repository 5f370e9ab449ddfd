"""Pins of the RoPE-shift / splice oracle (CPU).

- the cos/sin table against float64 math;
- shift_keys bit for bit against the reference's torch op sequence
  (threadcut/kv.py:20-25) on the same data;
- the T1 composition identity of the reference's tests (tests/test_core.py:67-74),
  with RoPE from transformers' own Qwen3 rotary embedding;
- shift(0) = identity, per-pair norms, shift(d1)∘shift(d2) ≈ shift(d1+d2);
- splice_growing vs splice_copy on the reference's known-answer splits
  (tests/test_core.py:104-121), vs a per-row brute force, rows outside
  [a, a+c) untouched; planted mistakes are caught.
"""
import numpy as np
import pytest
import torch
from transformers import Qwen3Config
from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding

from oracle import splice as osp
from oracle.decode import from_dtype_bits


def rope_at(rot, x, p):
    cos, sin = rot(x, torch.full((1, x.shape[2]), p, dtype=torch.long))
    x1, x2 = x[..., : x.shape[-1] // 2], x[..., x.shape[-1] // 2:]
    return x * cos[:, None].float() + torch.cat((-x2, x1), -1) * sin[:, None].float()


def keys16(seed, *shape):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)).half().numpy()


def test_inv_freq_matches_transformers():
    cfg = Qwen3Config(head_dim=128, rope_theta=1e6)
    rot = Qwen3RotaryEmbedding(cfg)
    assert torch.equal(osp.default_inv_freq(1e6, 128), rot.inv_freq.float())


@pytest.mark.parametrize("delta", [-6620, -350, -1, 0, 7, 131072])
def test_table_matches_float64(delta):
    inv = osp.default_inv_freq(1e6, 128)
    cos, sin = osp.rope_table(delta, inv)
    angle = np.float32(delta) * inv.numpy()  # the fp32 product, as the reference forms it
    assert np.abs(cos - np.cos(angle.astype(np.float64))).max() < 2e-7
    assert np.abs(sin - np.sin(angle.astype(np.float64))).max() < 2e-7


@pytest.mark.parametrize("delta", [-6620, -350, 1234])
def test_shift_bit_exact_vs_reference_op_sequence(delta):
    inv = osp.default_inv_freq(1e6, 128)
    k = keys16(1, 1, 8, 300, 128)
    cos, sin = osp.rope_table(delta, inv)
    got = osp.shift_keys(k, cos, sin)
    # threadcut/kv.py:20-25 op for op, on the CPU.
    kt = torch.from_numpy(k)
    angle = delta * inv.float()
    emb = torch.cat((angle, angle))
    kf = kt.float()
    x1, x2 = kf.chunk(2, dim=-1)
    ref = (kf * emb.cos() + torch.cat((-x2, x1), dim=-1) * emb.sin()).to(kt.dtype)
    assert np.array_equal(got.view(np.uint16), ref.numpy().view(np.uint16))


def test_shift_bf16_bit_exact_vs_torch():
    inv = osp.default_inv_freq(1e6, 128)
    kt = torch.randn(2, 4, 50, 128, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    cos, sin = osp.rope_table(-777, inv)
    got = osp.shift_keys(kt.view(torch.int16).numpy().view(np.uint16), cos, sin, dtype="bfloat16")
    angle = -777 * inv.float()
    emb = torch.cat((angle, angle))
    kf = kt.float()
    x1, x2 = kf.chunk(2, dim=-1)
    ref = (kf * emb.cos() + torch.cat((-x2, x1), dim=-1) * emb.sin()).to(torch.bfloat16)
    assert np.array_equal(got, ref.view(torch.int16).numpy().view(np.uint16))


@pytest.mark.parametrize("head_dim,theta", [(16, 1e4), (128, 1e6)])
def test_T1_composition(head_dim, theta):
    """shift(rope(k, 900), -350) == rope(k, 550) in fp32 math (atol 1e-4 as in the reference)."""
    rot = Qwen3RotaryEmbedding(Qwen3Config(head_dim=head_dim, rope_theta=theta, max_position_embeddings=4096))
    k = torch.randn(1, 2, 5, head_dim, generator=torch.Generator().manual_seed(3))
    cos, sin = osp.rope_table(-350, rot.inv_freq)
    x = rope_at(rot, k, 900).numpy()
    half = head_dim // 2
    x1, x2 = x[..., :half], x[..., half:]
    shifted = np.concatenate((x1 * cos - x2 * sin, x2 * cos + x1 * sin), -1)
    assert np.abs(shifted - rope_at(rot, k, 550).numpy()).max() < 1e-4


def test_shift_invariants():
    inv = osp.default_inv_freq(1e6, 128)
    k = keys16(4, 1, 8, 64, 128)
    c0, s0 = osp.rope_table(0, inv)
    assert np.array_equal(osp.shift_keys(k, c0, s0).view(np.uint16), k.view(np.uint16))
    c1, s1 = osp.rope_table(-300, inv)
    c2, s2 = osp.rope_table(-200, inv)
    c3, s3 = osp.rope_table(-500, inv)
    two = osp.shift_keys(osp.shift_keys(k, c1, s1), c2, s2).astype(np.float32)
    one = osp.shift_keys(k, c3, s3).astype(np.float32)
    assert np.abs(two - one).max() < 2e-2  # two fp16 roundings vs one
    kf = k.astype(np.float32)
    out = osp.shift_keys(k, c1, s1).astype(np.float32)
    norm_in = kf[..., :64] ** 2 + kf[..., 64:] ** 2
    norm_out = out[..., :64] ** 2 + out[..., 64:] ** 2
    assert np.abs(np.sqrt(norm_in) - np.sqrt(norm_out)).max() < 1e-2


def brute_splice(kbuf, vbuf, a, c0, c, cos, sin):
    kb, vb = kbuf.copy(), vbuf.copy()
    src_k = [kbuf[..., c0 + t, :].copy() for t in range(c)]
    src_v = [vbuf[..., c0 + t, :].copy() for t in range(c)]
    for t in range(c):
        row = src_k[t]
        if c0 != a:
            row = osp.shift_keys(row[..., None, :], cos, sin)[..., 0, :]
        kb[..., a + t, :] = row
        vb[..., a + t, :] = src_v[t]
    return kb, vb


@pytest.mark.parametrize("a,c0,c", [(10, 17, 20), (12, 12, 0), (0, 1, 39), (3, 30, 10), (5, 25, 15)])
def test_splice_growing_vs_copy_and_brute_force(a, c0, c):
    inv = osp.default_inv_freq(1e4, 128)
    k = keys16(5, 1, 2, 40, 128)
    v = keys16(6, 1, 2, 40, 128)
    cos, sin = osp.rope_table(-(c0 - a), inv)
    kb, vb, n = osp.splice_growing(k, v, 40, a, c0, c, cos, sin)
    ck, cv = osp.splice_copy(k, v, a, c0, c, cos, sin)
    assert n == a + c
    assert np.array_equal(kb[..., :n, :].view(np.uint16), ck.view(np.uint16))
    assert np.array_equal(vb[..., :n, :].view(np.uint16), cv.view(np.uint16))
    bk, bv = brute_splice(k, v, a, c0, c, cos, sin)
    assert np.array_equal(kb.view(np.uint16), bk.view(np.uint16))
    assert np.array_equal(vb.view(np.uint16), bv.view(np.uint16))
    # Rows outside [a, a + c) keep their contents.
    keep = np.r_[0:a, a + c:40]
    assert np.array_equal(kb[..., keep, :].view(np.uint16), k[..., keep, :].view(np.uint16))


def test_splice_keys_are_shifted_values_moved():
    """After a splice, C's keys equal RoPE at the new positions (fresh-compute identity, T2's core)."""
    rot = Qwen3RotaryEmbedding(Qwen3Config(head_dim=128, rope_theta=1e6, max_position_embeddings=8192))
    raw = torch.randn(1, 2, 30, 128, generator=torch.Generator().manual_seed(7))
    a, c0, c = 4, 19, 11
    cached = torch.cat([rope_at(rot, raw[:, :, t:t + 1], t) for t in range(30)], dim=2)
    fresh = torch.cat([rope_at(rot, raw[:, :, c0 + t:c0 + t + 1], a + t) for t in range(c)], dim=2)
    cos, sin = osp.rope_table(-(c0 - a), rot.inv_freq)
    kb, _, _ = osp.splice_growing(cached.half().numpy(), cached.half().numpy(), 30, a, c0, c, cos, sin)
    got = kb[..., a:a + c, :].astype(np.float32)
    assert np.abs(got - fresh.numpy()).max() < 2 * 2 ** -8


@pytest.mark.parametrize("mutation", ["no_rotation_sign", "wrong_source", "no_clone"])
def test_planted_mistakes_are_caught(mutation):
    inv = osp.default_inv_freq(1e4, 128)
    k = keys16(8, 1, 2, 40, 128)
    v = keys16(9, 1, 2, 40, 128)
    a, c0, c = 10, 17, 20
    cos, sin = osp.rope_table(-(c0 - a), inv)
    kb, vb = k.copy(), v.copy()
    if mutation == "no_rotation_sign":
        kk = from_dtype_bits(k[..., c0:c0 + c, :], "float16")
        lo = kk[..., :64] * cos + kk[..., 64:] * sin
        hi = kk[..., 64:] * cos + kk[..., :64] * sin
        kb[..., a:a + c, :] = np.concatenate((lo, hi), -1).astype(np.float16)
        vb[..., a:a + c, :] = v[..., c0:c0 + c, :]
    elif mutation == "wrong_source":
        kb[..., a:a + c, :] = osp.shift_keys(k[..., c0 - 1:c0 + c - 1, :], cos, sin)
        vb[..., a:a + c, :] = v[..., c0 - 1:c0 + c - 1, :]
    else:  # row-by-row in-place move without reading C first: overlapping rows get clobbered
        for t in range(c):
            kb[..., a + t, :] = osp.shift_keys(kb[..., c0 + t:c0 + t + 1, :], cos, sin)[..., 0, :]
            vb[..., a + t, :] = vb[..., c0 + t, :]
        # reverse order of traversal: a later source is overwritten first
        kb2, vb2 = k.copy(), v.copy()
        for t in reversed(range(c)):
            kb2[..., a + t, :] = osp.shift_keys(kb2[..., c0 + t:c0 + t + 1, :], cos, sin)[..., 0, :]
            vb2[..., a + t, :] = vb2[..., c0 + t, :]
        kb, vb = kb2, vb2
    ck, cv = osp.splice_copy(k, v, a, c0, c, cos, sin)
    same = np.array_equal(kb[..., :a + c, :].view(np.uint16), ck.view(np.uint16)) and \
        np.array_equal(vb[..., :a + c, :].view(np.uint16), cv.view(np.uint16))
    assert not same


@pytest.mark.parametrize("a,c0,c", [(10, 17, 20), (12, 12, 0), (5, 40, 24), (0, 3, 61)])
def test_torch_restatement_matches_numpy_oracle(a, c0, c):
    """The torch form of the reference's CPU splice (bench.py's splice baseline) is
    bit-identical to the numpy restatement, including overlapping moves."""
    inv = osp.default_inv_freq(1e6, 128)
    cos, sin = osp.rope_table(-(c0 - a), inv)
    k = torch.randn(1, 2, 64, 128, generator=torch.Generator().manual_seed(20)).half()
    v = torch.randn(1, 2, 64, 128, generator=torch.Generator().manual_seed(21)).half()
    kb, vb, _ = osp.splice_growing(k.numpy(), v.numpy(), 64, a, c0, c, cos, sin)
    kt, vt = [k.clone()], [v.clone()]
    osp.splice_growing_torch(kt, vt, a, c0, c, inv)
    assert np.array_equal(kt[0].numpy().view(np.uint16), kb.view(np.uint16))
    assert np.array_equal(vt[0].numpy().view(np.uint16), vb.view(np.uint16))
