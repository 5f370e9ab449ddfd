"""Pins of oracle.prefill: library routine, brute force, closed forms, mutations."""
import numpy as np
import pytest
import torch

from oracle import prefill as op


def draw(seed, b=2, hq=8, hkv=2, L=5, n=9, d=16):
    g = np.random.default_rng(seed)
    return (g.standard_normal((b, hq, L, d)), g.standard_normal((b, hkv, n, d)),
            g.standard_normal((b, hkv, n, d)))


def causal_past(L, n):
    return np.arange(n)[None, :] <= np.arange(L)[:, None] + (n - L)


def torch_sdpa64(q, k, v, scale, mask=None, causal=False):
    import torch.nn.functional as F

    g = q.shape[1] // k.shape[1]
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x))
    m = None if mask is None else t(np.asarray(mask, bool))
    out = F.scaled_dot_product_attention(t(q), t(k).repeat_interleave(g, 1), t(v).repeat_interleave(g, 1),
                                         attn_mask=m, scale=scale, is_causal=causal)
    return out.transpose(1, 2).numpy()


@pytest.mark.parametrize("seed", range(4))
def test_against_torch_sdpa(seed):
    q, k, v = draw(seed)
    s = 0.37
    np.testing.assert_allclose(op.prefill_f64(q, k, v, s), torch_sdpa64(q, k, v, s), atol=1e-12)
    qc, kc, vc = draw(seed, L=9, n=9)
    np.testing.assert_allclose(op.prefill_f64(qc, kc, vc, s, causal=True),
                               torch_sdpa64(qc, kc, vc, s, causal=True), atol=1e-12)
    m = causal_past(5, 9)[None, None].repeat(2, 0)
    np.testing.assert_allclose(op.prefill_f64(q, k, v, s, mask=m), torch_sdpa64(q, k, v, s, mask=m), atol=1e-12)
    r = np.random.default_rng(seed).random((2, 1, 5, 9)) < 0.6
    r[..., 0] = True
    np.testing.assert_allclose(op.prefill_f64(q, k, v, s, mask=r), torch_sdpa64(q, k, v, s, mask=r), atol=1e-12)


def brute(q, k, v, scale, vis):
    b, hq, L, d = q.shape
    g = hq // k.shape[1]
    out = np.zeros((b, L, hq, d))
    for bi in range(b):
        for h in range(hq):
            for t in range(L):
                js = [j for j in range(k.shape[2]) if vis[bi, t, j]]
                if not js:
                    continue
                sc = [sum(q[bi, h, t, e] * k[bi, h // g, j, e] for e in range(d)) * scale for j in js]
                mx = max(sc)
                w = [np.exp(x - mx) for x in sc]
                for e in range(d):
                    out[bi, t, h, e] = sum(wi * v[bi, h // g, j, e] for wi, j in zip(w, js)) / sum(w)
    return out


def test_brute_force_tiny():
    q, k, v = draw(7, b=1, hq=4, hkv=2, L=3, n=5, d=4)
    m = np.random.default_rng(1).random((1, 1, 3, 5)) < 0.5
    m[0, 0, 1] = False  # a row with no visible key -> zeros
    for kw in ({}, {"causal": True}, {"mask": m}):
        vis = op.visible(3, 5, kw.get("mask"), kw.get("causal", False), 1)
        np.testing.assert_allclose(op.prefill_f64(q, k, v, 0.5, **kw), brute(q, k, v, 0.5, vis), atol=1e-12)
    assert np.all(op.prefill_f64(q, k, v, 0.5, mask=m)[0, 1] == 0)


def test_closed_forms():
    q, k, v = draw(3, b=1, hq=4, hkv=1, L=4, n=6)
    one = np.zeros((1, 1, 4, 6), bool)
    one[..., 2] = True
    out = op.prefill_f64(q, k, v, 1.0, mask=one)
    assert np.allclose(out, v[0, 0, 2][None, None, None, :])
    vc = np.broadcast_to(v[:, :, :1], v.shape)
    assert np.allclose(op.prefill_f64(q, k, vc, 1.0, causal=True), v[0, 0, 0][None, None, None, :])
    out = op.prefill_f64(np.zeros_like(q), k, v, 1.0, causal=True)
    for t in range(4):
        assert np.allclose(out[0, t, 0], v[0, 0, :t + 3].mean(0))  # past = 2
    qq, kq, vq = draw(4, b=1, hq=2, hkv=1, L=6, n=6)
    assert np.allclose(op.prefill_f64(qq, kq, vq, 1.0, causal=True)[0, 0], vq[0, 0, 0])
    allm = np.ones((1, 1, 4, 6), bool)
    assert np.array_equal(op.prefill_f64(q, k, v, 0.2, mask=allm), op.prefill_f64(q, k, v, 0.2))


def test_mutations_fail_the_pins():
    q, k, v = draw(11, b=1, hq=8, hkv=2, L=6, n=6)
    good = torch_sdpa64(q, k, v, 0.3, causal=True)
    # heads mapped h + i*hkv instead of h*g + i
    kk = np.concatenate([k, k, k, k], axis=1)
    vv = np.concatenate([v, v, v, v], axis=1)
    assert not np.allclose(op.prefill_f64(q, kk, vv, 0.3, causal=True), good, atol=1e-3)
    # causal triangle off by one
    m = causal_past(6, 6)
    off = np.roll(m, 1, axis=1)
    off[0] = m[0]
    assert not np.allclose(op.prefill_f64(q, k, v, 0.3, mask=off[None, None]), good, atol=1e-3)
    # transposed mask
    r = np.random.default_rng(2).random((6, 6)) < 0.5
    np.fill_diagonal(r, True)
    assert not np.allclose(op.prefill_f64(q, k, v, 0.3, mask=r.T[None, None]),
                           torch_sdpa64(q, k, v, 0.3, mask=r[None, None]), atol=1e-3)


def test_sdpa_reference_is_the_oracle():
    q, k, v = draw(5, b=1, hq=8, hkv=2, L=7, n=7)
    t = lambda x: torch.from_numpy(x)
    np.testing.assert_allclose(op.sdpa_reference(t(q), t(k), t(v), None, 0.25).numpy(),
                               op.prefill_f64(q, k, v, 0.25, causal=True), atol=1e-12)
