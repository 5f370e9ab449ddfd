"""Pins of the decode oracle (CPU): closed form, library SDPA, brute force, invariants.

Each check is chosen so that a plausible mistake in a restatement of
threadcut/flash_decode.py:21-69 fails it; the mutation tests at the end plant
such mistakes in a copy of the oracle and show the pins catch them.
"""
import numpy as np
import pytest
import torch

from oracle import decode as od

SCALE = 128 ** -0.5


def rand(seed, *shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def brute_force(q, k, v, scale):
    """Pure-Python loops over a tiny shape: exp/sum per query row, float64."""
    hkv, g, d = q.shape
    n = k.shape[1]
    out = np.zeros((hkv, g, d))
    for h in range(hkv):
        for i in range(g):
            s = [sum(float(q[h, i, e]) * float(k[h, t, e]) for e in range(d)) * scale for t in range(n)]
            mx = max(s)
            w = [np.exp(x - mx) for x in s]
            tot = sum(w)
            for e in range(d):
                out[h, i, e] = sum(w[t] * float(v[h, t, e]) for t in range(n)) / tot
    return out


def test_closed_form_matches_brute_force():
    q, k, v = rand(1, 2, 3, 8), rand(2, 2, 11, 8), rand(3, 2, 11, 8)
    assert np.abs(od.attention_f64(q, k, v, 0.3) - brute_force(q, k, v, 0.3)).max() < 1e-12


@pytest.mark.parametrize("n", [1, 7, 16, 17, 255, 256, 257, 700, 1536])
def test_split_kv_matches_closed_form(n):
    q, k, v = rand(4, 8, 4, 128), rand(5, 8, n, 128), rand(6, 8, n, 128)
    got = od.decode_attention(q, k, v, SCALE)
    assert np.abs(got - od.attention_f64(q, k, v, SCALE)).max() < 2e-6


def test_split_kv_matches_torch_sdpa():
    """Library pin: torch's own SDPA (fp32, CPU) on the folded-GQA decode shape."""
    q = torch.from_numpy(rand(7, 1, 32, 1, 128))
    k = torch.from_numpy(rand(8, 1, 8, 1536, 128))
    v = torch.from_numpy(rand(9, 1, 8, 1536, 128))
    sdpa = od.folded_sdpa(q, k, v, SCALE).reshape(8, 4, 128).numpy()
    got = od.decode_attention(q.numpy().reshape(8, 4, 128), k[0].numpy(), v[0].numpy(), SCALE)
    assert np.abs(got - sdpa).max() < 2e-6


def test_folded_sdpa_is_per_head_attention():
    """The folding of attention.py:41 maps query head h*g+i to KV head h."""
    q = torch.from_numpy(rand(10, 2, 8, 1, 64))
    k = torch.from_numpy(rand(11, 2, 2, 33, 64))
    v = torch.from_numpy(rand(12, 2, 2, 33, 64))
    got = od.folded_sdpa(q, k, v, 0.2)
    for b in range(2):
        for hq in range(8):
            h = hq // 4
            want = od.attention_f64(q[b, hq].numpy(), k[b, h].numpy(), v[b, h].numpy(), 0.2)
            assert np.abs(got[b, hq].numpy() - want).max() < 1e-6


@pytest.mark.parametrize("split,block", [(16, 16), (64, 16), (256, 16), (4096, 16), (256, 32)])
def test_split_length_does_not_change_result(split, block):
    q, k, v = rand(13, 4, 4, 128), rand(14, 4, 1000, 128), rand(15, 4, 1000, 128)
    a = od.decode_attention(q, k, v, SCALE, split=split, block=block)
    b = od.decode_attention(q, k, v, SCALE, split=1024, block=16)
    assert np.abs(a - b).max() < 2e-6


def test_single_split_combine_is_identity():
    q, k, v = rand(16, 2, 4, 128), rand(17, 2, 100, 128), rand(18, 2, 100, 128)
    o, lse = od.flash_decode_partial(q, k, v, SCALE, split=256)
    assert o.shape[0] == 1
    assert np.array_equal(od.flash_decode_combine(o, lse), o[0])


def test_lse_is_log_partition():
    q, k, v = rand(19, 2, 4, 128), rand(20, 2, 300, 128), rand(21, 2, 300, 128)
    o, lse = od.flash_decode_partial(q, k, v, SCALE, split=256)
    s = np.einsum("hgd,hnd->hgn", q.astype(np.float64), k.astype(np.float64)) * SCALE
    want0 = np.log(np.exp(s[:, :, :256]).sum(-1))
    want1 = np.log(np.exp(s[:, :, 256:]).sum(-1))
    assert np.abs(lse[0] - want0).max() < 1e-5 and np.abs(lse[1] - want1).max() < 1e-5


def test_constant_values_and_zero_query():
    q, k, v = rand(22, 2, 4, 128), rand(23, 2, 500, 128), rand(24, 2, 500, 128)
    v[:] = v[:, 3:4]
    assert np.abs(od.decode_attention(q, k, v, SCALE) - v[:, 3][:, None]).max() < 1e-6
    v = rand(25, 2, 500, 128)
    got = od.decode_attention(np.zeros_like(q), k, v, SCALE)
    assert np.abs(got - v.mean(axis=1)[:, None]).max() < 1e-6


def test_empty_cache_is_zero():
    q = rand(26, 8, 4, 128)
    empty = np.zeros((8, 0, 128), np.float32)
    assert np.array_equal(od.decode_attention(q, empty, empty, SCALE), np.zeros((8, 4, 128), np.float32))


def test_large_scores_stay_finite():
    q, k, v = rand(27, 2, 4, 128, scale=30.0), rand(28, 2, 800, 128), rand(29, 2, 800, 128)
    got = od.decode_attention(q, k, v, SCALE)
    assert np.isfinite(got).all()
    assert np.abs(got - od.attention_f64(q, k, v, SCALE)).max() < 1e-4


def test_ragged_uses_only_valid_rows():
    q, k, v = rand(30, 3, 2, 4, 16), rand(31, 3, 2, 50, 16), rand(32, 3, 2, 50, 16)
    lens = np.array([50, 7, 0])
    got = od.decode_ragged(q, k, v, lens, 0.25)
    k2, v2 = k.copy(), v.copy()
    k2[1, :, 7:] = 1e4
    v2[1, :, 7:] = np.nan
    assert np.array_equal(od.decode_ragged(q, k2, v2, lens, 0.25), got)
    assert np.all(got[2] == 0)


def test_bf16_rounding_is_nearest_even():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, np.inf, np.nan], np.float32)
    bits = od.to_dtype_bits(x, "bfloat16")
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bits[:5], want[:5]) and np.isnan(od.from_dtype_bits(bits[5:], "bfloat16")).all()


# --- planted mistakes: each mutated oracle must fail at least one pin above ---

def _mutant_partial(q, k, v, scale, split=256, block=16, mutation=None):
    hkv, g, d = q.shape
    n = k.shape[1]
    S = -(-n // split)
    o = np.empty((S, hkv, g, d), np.float32)
    lse = np.empty((S, hkv, g), np.float32)
    for s in range(S):
        m = np.full((hkv, g), -np.inf, np.float32)
        l = np.zeros((hkv, g), np.float32)
        acc = np.zeros((hkv, g, d), np.float32)
        for off in range(s * split, s * split + split, block):
            idx = off + np.arange(block)
            valid = idx < n
            kb = np.zeros((hkv, block, d), np.float32)
            vb = np.zeros((hkv, block, d), np.float32)
            kb[:, valid] = k[:, idx[valid]]
            vb[:, valid] = v[:, idx[valid]]
            if mutation == "transpose_v":
                vb = vb[:, ::-1]
            qk = np.einsum("hgd,hnd->hgn", q, kb) * scale
            if mutation != "no_mask":
                qk = np.where(valid[None, None, :], qk, -np.inf)
            m_new = np.maximum(m, qk.max(axis=2))
            m_safe = np.where(m_new == -np.inf, 0, m_new)
            p = np.exp(qk - m_safe[:, :, None])
            alpha = np.exp(m - m_safe)
            if mutation == "no_rescale":
                alpha = np.ones_like(alpha)
            l = l * alpha + p.sum(axis=2)
            acc = acc * alpha[:, :, None] + np.einsum("hgn,hnd->hgd", p, vb)
            m = m_new
        o[s] = acc / np.where(l == 0, 1, l)[:, :, None]
        lse[s] = np.where(l == 0, -np.inf, m + np.log(l))
        if mutation == "lse_log2":
            lse[s] = np.where(l == 0, -np.inf, m + np.log2(l))
    return o, lse


@pytest.mark.parametrize("mutation", ["no_rescale", "no_mask", "transpose_v", "lse_log2"])
def test_planted_mistakes_are_caught(mutation):
    q, k, v = rand(33, 2, 4, 128, scale=3.0), rand(34, 2, 600, 128), rand(35, 2, 600, 128)
    with np.errstate(all="ignore"):
        o, lse = _mutant_partial(q, k, v, SCALE, mutation=mutation)
        got = od.flash_decode_combine(o, lse)
    assert not np.abs(got - od.attention_f64(q, k, v, SCALE)).max() < 2e-6
