"""Decode parity on the GPU: HIP kernels vs the CPU oracle on the same seeded inputs.

Tolerance (fp16/bf16 outputs after fp32 accumulation): max-abs 2e-3 against
the float64 closed form / fp32 SDPA; fp32 partials within 1e-4 of the
restated split-KV kernel at the same split length.
"""
import numpy as np
import pytest
import torch

from oracle import decode as od
from threadcut_amd import _lib, attention, flash_decode, workloads

pytestmark = pytest.mark.gpu

TOL = 2e-3
SCALE = 128 ** -0.5


def f64_ref(q, k, v, scale=SCALE, lens=None):
    """q [B,Hq,1,D] torch (cpu), k/v [B,Hkv,N,D] -> float64 [B,Hkv,G,D]."""
    b, hq, _, d = q.shape
    hkv = k.shape[1]
    qn = q.float().numpy().reshape(b, hkv, hq // hkv, d)
    kn, vn = k.float().numpy(), v.float().numpy()
    if lens is None:
        return od.attention_f64(qn, kn, vn, scale)
    return od.decode_ragged(qn, kn, vn, lens.numpy(), scale)


def run_decode(q, k, v, dev, scale=SCALE, lens=None, split=None):
    b, hq, _, d = q.shape
    hkv = k.shape[1]
    qd = q.to(dev).reshape(b, hkv, hq // hkv, d)
    out = flash_decode.decode_attention_batched(qd, k.to(dev), v.to(dev), scale,
                                                lens=None if lens is None else lens.to(dev), split=split)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def test_single_call_shape_vs_fp32_sdpa(gpu):
    """Q [1,32,1,128], K/V [1,8,1536,128] fp16, seed 0, against torch SDPA in fp32."""
    q, k, v, _ = workloads.decode_inputs(0, n=1536)
    print("case: single call n=1536 seed 0", flush=True)
    out, none = attention.attention(None, q.to(gpu), k.to(gpu), v.to(gpu), None, scaling=SCALE)
    torch.cuda.synchronize()
    assert none is None and out.shape == (1, 1, 32, 128) and out.is_contiguous()
    ref = od.folded_sdpa(q.float(), k.float(), v.float(), SCALE).transpose(1, 2)
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= TOL, err
    ref64 = f64_ref(q, k, v).reshape(1, 1, 32, 128)
    assert np.abs(out.float().cpu().numpy() - ref64).max() <= TOL


@pytest.mark.parametrize("n", [1, 2, 15, 16, 17, 63, 64, 65, 100, 255, 256, 257, 1000, 1536, 4096])
@pytest.mark.parametrize("split", [None, 64, 256])
def test_lengths_and_splits(gpu, n, split):
    q, k, v, _ = workloads.decode_inputs(100 + n, n=n)
    print(f"case: n={n} split={split}", flush=True)
    got = run_decode(q, k, v, gpu, split=split)
    assert np.abs(got - f64_ref(q, k, v)).max() <= TOL


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (24, 8), (32, 8), (40, 8), (64, 8), (32, 4), (14, 2)])
def test_group_sizes(gpu, hq, hkv):
    q, k, v, _ = workloads.decode_inputs(7, n=777, q_heads=hq, kv_heads=hkv)
    print(f"case: hq={hq} hkv={hkv}", flush=True)
    got = run_decode(q, k, v, gpu)
    assert np.abs(got - f64_ref(q, k, v)).max() <= TOL


def test_bf16(gpu):
    q, k, v, _ = workloads.decode_inputs(8, n=3000, dtype=torch.bfloat16)
    got = run_decode(q, k, v, gpu)
    # bf16 output rounding: half an ulp of bf16 at |out| < 1 is 2^-9.
    assert np.abs(got - f64_ref(q, k, v)).max() <= 4e-3


def test_partials_match_restated_kernel(gpu):
    """o_part / lse_part at split 256 against the restated Triton program."""
    q, k, v, _ = workloads.decode_inputs(9, n=1000)
    hkv, g, d = 8, 4, 128
    qd = q.to(gpu).reshape(1, hkv, g, d)
    kd, vd = k.to(gpu), v.to(gpu)
    S = flash_decode.num_splits(1, hkv, 1000, 256)
    assert S == 4
    o = torch.empty((1, hkv, S, g, d), dtype=torch.float32, device=gpu)
    lse = torch.empty((1, hkv, S, g), dtype=torch.float32, device=gpu)
    lib = _lib.load()
    rc = lib.tc_decode_partial(qd.data_ptr(), _lib.i64x3(*qd.stride()[:3]), kd.data_ptr(), _lib.i64x3(*kd.stride()[:3]),
                               vd.data_ptr(), _lib.i64x3(*vd.stride()[:3]), None, 1000, 1, hkv, g, d,
                               _lib.TC_DTYPE_F16, SCALE, 256, S, o.data_ptr(), lse.data_ptr(),
                               _lib.stream_of(gpu))
    _lib.check(rc, "tc_decode_partial")
    torch.cuda.synchronize()
    ro, rl = od.flash_decode_partial(q.float().numpy().reshape(hkv, g, d), k[0].float().numpy(),
                                     v[0].float().numpy(), SCALE, split=256)
    assert np.abs(o[0].permute(1, 0, 2, 3).cpu().numpy() - ro).max() <= 1e-4
    assert np.abs(lse[0].permute(1, 0, 2).cpu().numpy() - rl).max() <= 1e-4
    # Combine alone on the oracle's partials.
    out = torch.empty((1, hkv, g, d), dtype=torch.float16, device=gpu)
    o2 = torch.from_numpy(ro).permute(1, 0, 2, 3).contiguous()[None].to(gpu)
    l2 = torch.from_numpy(rl).permute(1, 0, 2).contiguous()[None].to(gpu)
    rc = lib.tc_decode_combine(o2.data_ptr(), l2.data_ptr(), 1, hkv, g, d, S, out.data_ptr(),
                               _lib.i64x3(*out.stride()[:3]), _lib.TC_DTYPE_F16, _lib.stream_of(gpu))
    _lib.check(rc, "tc_decode_combine")
    torch.cuda.synchronize()
    comb = od.flash_decode_combine(ro, rl)
    assert np.abs(out[0].float().cpu().numpy() - comb).max() <= 1e-3


def test_empty_cache_gives_zeros(gpu):
    q, k, v, _ = workloads.decode_inputs(10, n=0)
    got = run_decode(q, k, v, gpu)
    assert got.shape == (1, 8, 4, 128) and np.all(got == 0)


def test_strided_cache_views_and_transposed_query(gpu):
    """K/V as views [..., :n, :] of a larger buffer; q as the transposed [b, hq, 1, d] view."""
    cap, n = 5000, 3333
    g_ = torch.Generator().manual_seed(11)
    kbuf = torch.randn(1, 8, cap, 128, generator=g_).half().to(gpu)
    vbuf = torch.randn(1, 8, cap, 128, generator=g_).half().to(gpu)
    qflat = torch.randn(1, 1, 32, 128, generator=g_).half().to(gpu)
    query = qflat.transpose(1, 2)  # [1, 32, 1, 128], strides of a transpose
    out, _ = attention.attention(None, query, kbuf[:, :, :n], vbuf[:, :, :n], None, scaling=SCALE)
    torch.cuda.synchronize()
    ref = f64_ref(query.cpu(), kbuf[:, :, :n].cpu(), vbuf[:, :, :n].cpu()).reshape(1, 1, 32, 128)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= TOL


def test_large_scores_stay_finite(gpu):
    """q scaled by 10: scores of ~N(0, 100), a peaked softmax."""
    q, k, v, _ = workloads.decode_inputs(12, n=2048)
    q = (q.float() * 10).half()
    got = run_decode(q, k, v, gpu)
    assert np.isfinite(got).all()
    assert np.abs(got - f64_ref(q, k, v)).max() <= TOL


def test_constant_values_and_zero_query(gpu):
    q, k, v, _ = workloads.decode_inputs(13, n=900)
    v_const = v.clone()
    v_const[:] = v[:, :, 5:6, :]
    got = run_decode(q, k, v_const, gpu)
    row = v[:, :, 5, :].float().numpy()[:, :, None, :]
    assert np.abs(got - row).max() <= TOL
    got0 = run_decode(torch.zeros_like(q), k, v, gpu)
    mean = v.float().numpy().mean(axis=2)[:, :, None, :]
    assert np.abs(got0 - mean).max() <= TOL


def test_ragged_batch_sixteen_sequences(gpu):
    """16 sequences, lengths U[1024, 32768] (seed 3), padded cache + int32 lengths."""
    q, k, v, lens = workloads.decode_inputs(3, batch=16, n=32768, lens_range=(1024, 32768))
    print(f"case: ragged B=16 lens={lens.tolist()}", flush=True)
    got = run_decode(q, k, v, gpu, lens=lens)
    ref = f64_ref(q, k, v, lens=lens)
    assert np.abs(got - ref).max() <= TOL


def test_ragged_with_empty_and_full_rows(gpu):
    q, k, v, _ = workloads.decode_inputs(14, batch=4, n=700)
    lens = torch.tensor([0, 1, 699, 700], dtype=torch.int32)
    got = run_decode(q, k, v, gpu, lens=lens)
    ref = f64_ref(q, k, v, lens=lens)
    assert np.all(got[0] == 0)
    assert np.abs(got - ref).max() <= TOL


@pytest.mark.parametrize("lens", [[300, 300, 300, 300, 300, 300], [0, 513, 0, 513, 64, 64, 700],
                                  [700 - (i % 5) * 100 for i in range(64)], [5 * (i % 3) for i in range(33)]])
def test_ragged_longest_first_covers_every_sequence(gpu, lens):
    """With per-sequence lengths the partial serves the sequences longest first (grid row z takes
    the z-th longest, ties by index): ties, empty rows and 64 sequences must still give every
    sequence exactly its own splits."""
    print(f"case: ragged longest-first B={len(lens)} lens={lens[:8]}...", flush=True)
    q, k, v, _ = workloads.decode_inputs(15, batch=len(lens), n=700)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    got = run_decode(q, k, v, gpu, lens=lens_t)
    ref = f64_ref(q, k, v, lens=lens_t)
    assert np.abs(got - ref).max() <= TOL


@pytest.mark.parametrize("batch", [1, 4])
def test_long_context_131072(gpu, batch):
    """131072 tokens (seed 4): many splits and the LSE combine, vs fp32 SDPA on the CPU."""
    q, k, v, _ = workloads.decode_inputs(4, batch=batch, n=131072)
    print(f"case: long context B={batch} n=131072", flush=True)
    got = run_decode(q, k, v, gpu)
    ref = od.folded_sdpa(q.float(), k.float(), v.float(), SCALE).reshape(batch, 8, 4, 128).numpy()
    assert np.abs(got - ref).max() <= TOL


def test_decode_attention_signature(gpu):
    """flash_decode.decode_attention(q [hkv,g,d], k, v [hkv,n,d], scale, split, block)."""
    q, k, v, _ = workloads.decode_inputs(15, n=1300)
    out = flash_decode.decode_attention(q.to(gpu).reshape(8, 4, 128), k[0].to(gpu), v[0].to(gpu), SCALE,
                                        split=256, block=16)
    torch.cuda.synchronize()
    assert out.shape == (8, 4, 128) and out.dtype == torch.float16
    assert np.abs(out.float().cpu().numpy() - f64_ref(q, k, v)[0]).max() <= TOL


def test_rejects_bad_inputs(gpu):
    q, k, v, _ = workloads.decode_inputs(16, n=64, head_dim=64)
    with pytest.raises(RuntimeError, match="head_dim"):
        run_decode(q, k, v, gpu)
    q, k, v, _ = workloads.decode_inputs(16, n=64)
    with pytest.raises(RuntimeError, match="GPU"):
        flash_decode.decode_attention(q.reshape(8, 4, 128), k[0], v[0], SCALE)


@pytest.mark.parametrize("n", [1, 2, 17, 1501, 10240])
def test_append_attention_writes_the_row_and_attends_over_it(gpu, n):
    """tc_decode_append_attention: new K/V row written at n - 1, output as if it were in the cache."""
    cap = n + 37
    q, k, v, _ = workloads.decode_inputs(30 + n, n=cap)
    g_ = torch.Generator().manual_seed(31)
    k_new = torch.randn(1, 8, 1, 128, generator=g_).half()
    v_new = torch.randn(1, 8, 1, 128, generator=g_).half()
    kc, vc = k.to(gpu), v.to(gpu)
    out = torch.empty((1, 8, 4, 128), dtype=torch.float16, device=gpu)
    flash_decode.decode_append_into(q.to(gpu).reshape(1, 8, 4, 128), kc, vc, k_new.to(gpu), v_new.to(gpu), n,
                                    SCALE, out)
    torch.cuda.synchronize()
    k_ref, v_ref = k.clone(), v.clone()
    k_ref[:, :, n - 1] = k_new[:, :, 0]
    v_ref[:, :, n - 1] = v_new[:, :, 0]
    assert torch.equal(kc.cpu(), k_ref) and torch.equal(vc.cpu(), v_ref)   # only row n - 1 changed
    ref = f64_ref(q, k_ref[:, :, :n], v_ref[:, :, :n])
    assert np.abs(out.float().cpu().numpy() - ref).max() <= TOL



@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_softmax_weights_are_not_rounded_to_the_element_type(gpu, dtype):
    """Two visible tokens with weights 1 and p1 = e^(b1 - 4), b1 chosen so that p1 is far
    from a value of the element type: the fp32 partial must keep that weight (the
    matrix-core P.V adds the rounding residue of P as a second product). Rounded P
    alone would be off by up to 2^-9 (bf16) or 2^-12 (fp16) relative; the bar is 1e-5."""
    hkv, g, d, n = 8, 4, 128, 64
    # b1 on the element type's grid in [3, 4) whose weight e^(b1 - 4) rounds worst.
    cand = torch.arange(3.0, 4.0, 1 / 64, dtype=torch.float64).to(dtype).double().unique()
    p1 = torch.exp(cand - 4.0)
    err = (p1 - p1.to(dtype).double()).abs() / p1
    b1 = float(cand[int(err.argmax())])
    p1 = float(torch.exp(torch.tensor(b1 - 4.0, dtype=torch.float64)))
    q = torch.zeros(1, hkv, g, d, dtype=dtype)
    q[..., 0] = 1.0
    k = torch.zeros(1, hkv, n, d, dtype=dtype)
    k[..., 0] = -64.0          # every other key: weight e^-68, nothing in fp32 next to 1
    k[:, :, 5, 0] = 4.0
    k[:, :, 9, 0] = b1
    v = torch.zeros(1, hkv, n, d, dtype=dtype)
    v[:, :, 5] = 1.0
    v[:, :, 9] = -1.0
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    o = torch.empty((1, hkv, 1, g, d), dtype=torch.float32, device=gpu)
    lse = torch.empty((1, hkv, 1, g), dtype=torch.float32, device=gpu)
    lib = _lib.load()
    rc = lib.tc_decode_partial(qd.data_ptr(), _lib.i64x3(*qd.stride()[:3]), kd.data_ptr(), _lib.i64x3(*kd.stride()[:3]),
                               vd.data_ptr(), _lib.i64x3(*vd.stride()[:3]), None, n, 1, hkv, g, d,
                               _lib.dtype_code(dtype), 1.0, 64, 1, o.data_ptr(), lse.data_ptr(), _lib.stream_of(gpu))
    _lib.check(rc, "tc_decode_partial")
    torch.cuda.synchronize()
    want = (1.0 - p1) / (1.0 + p1)
    assert (o.cpu().double() - want).abs().max().item() <= 1e-5
    assert (lse.cpu().double() - (4.0 + np.log1p(p1))).abs().max().item() <= 1e-5


def test_nan_past_the_length_is_never_read(gpu):
    """Cache buffers hold NaN past the valid rows: views [..., :n, :] and per-sequence
    lengths only ever read valid rows (the loads' buffer range ends there)."""
    cap = 4096
    g_ = torch.Generator().manual_seed(61)
    kbuf = torch.full((3, 8, cap, 128), float("nan"), dtype=torch.float16)
    vbuf = torch.full((3, 8, cap, 128), float("nan"), dtype=torch.float16)
    lens = torch.tensor([1, 1000, 3001], dtype=torch.int32)
    for b_, n_ in enumerate(lens.tolist()):
        kbuf[b_, :, :n_] = torch.randn(8, n_, 128, generator=g_).half()
        vbuf[b_, :, :n_] = torch.randn(8, n_, 128, generator=g_).half()
    q = torch.randn(3, 32, 1, 128, generator=g_).half()
    got = run_decode(q, kbuf, vbuf, gpu, lens=lens)
    assert np.isfinite(got).all()
    assert np.abs(got - f64_ref(q, kbuf, vbuf, lens=lens)).max() <= TOL
    n = 1000
    kd, vd = kbuf.to(gpu), vbuf.to(gpu)   # slice on the device: the view's rows past n are NaN
    out = flash_decode.decode_attention_batched(q[1:2].to(gpu).reshape(1, 8, 4, 128), kd[1:2, :, :n],
                                                vd[1:2, :, :n], SCALE)
    torch.cuda.synchronize()
    ref = f64_ref(q[1:2], kbuf[1:2, :, :n], vbuf[1:2, :, :n])
    assert np.abs(out.float().cpu().numpy() - ref).max() <= TOL


def test_append_bf16_eight_query_heads_per_kv_head(gpu):
    """The fused append at g = 8 (64 query heads over 8 KV heads) in bf16."""
    n, cap = 2500, 2600
    q, k, v, _ = workloads.decode_inputs(62, n=cap, q_heads=64, dtype=torch.bfloat16)
    g_ = torch.Generator().manual_seed(63)
    k_new = torch.randn(1, 8, 1, 128, generator=g_).to(torch.bfloat16)
    v_new = torch.randn(1, 8, 1, 128, generator=g_).to(torch.bfloat16)
    kc, vc = k.to(gpu), v.to(gpu)
    out = torch.empty((1, 8, 8, 128), dtype=torch.bfloat16, device=gpu)
    flash_decode.decode_append_into(q.to(gpu).reshape(1, 8, 8, 128), kc, vc, k_new.to(gpu), v_new.to(gpu), n,
                                    SCALE, out)
    torch.cuda.synchronize()
    k_ref, v_ref = k.clone(), v.clone()
    k_ref[:, :, n - 1] = k_new[:, :, 0]
    v_ref[:, :, n - 1] = v_new[:, :, 0]
    assert torch.equal(kc.cpu(), k_ref) and torch.equal(vc.cpu(), v_ref)
    ref = f64_ref(q, k_ref[:, :, :n], v_ref[:, :, :n])
    assert np.abs(out.float().cpu().numpy() - ref).max() <= 4e-3


def test_gate_sends_supported_calls_to_the_kernels(gpu, monkeypatch):
    """fp16 and bf16 calls at head_dim 128 run the HIP kernels, never SDPA."""

    def no_sdpa(*a, **k):
        raise AssertionError("SDPA called for a call the kernels take")

    monkeypatch.setattr(attention.F, "scaled_dot_product_attention", no_sdpa)
    for dtype, tol in ((torch.float16, TOL), (torch.bfloat16, 4e-3)):
        q, k, v, _ = workloads.decode_inputs(41, n=300, dtype=dtype)
        print(f"case: gate {dtype} n=300", flush=True)
        out, _ = attention.attention(None, q.to(gpu), k.to(gpu), v.to(gpu), None, scaling=SCALE)
        torch.cuda.synchronize()
        ref = f64_ref(q, k, v).reshape(1, 1, 32, 128)
        assert np.abs(out.float().cpu().numpy() - ref).max() <= tol


@pytest.mark.parametrize("dtype,d,hq,hkv", [(torch.float32, 128, 32, 8), (torch.float16, 64, 32, 8),
                                            (torch.float16, 128, 32, 2)])
def test_gate_keeps_the_reference_path_for_other_calls(gpu, monkeypatch, dtype, d, hq, hkv):
    """float32, head_dim 64 and 16 query heads per KV head are not kernel shapes: the reference's
    folded SDPA runs on the GPU tensors (threadcut/attention.py:40-42), not the kernels."""

    def no_kernel(*a, **k):
        raise AssertionError("decode kernel called for a call it does not take")

    monkeypatch.setattr(attention, "decode_into", no_kernel)
    q, k, v, _ = workloads.decode_inputs(42, n=200, q_heads=hq, kv_heads=hkv, head_dim=d, dtype=dtype)
    print(f"case: gate {dtype} d={d} hq={hq} hkv={hkv}", flush=True)
    out, _ = attention.attention(None, q.to(gpu), k.to(gpu), v.to(gpu), None, scaling=d ** -0.5)
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == (1, 1, hq, d) and out.is_contiguous()
    ref = od.attention_f64(q.float().numpy().reshape(1, hkv, hq // hkv, d), k.float().numpy(), v.float().numpy(),
                           d ** -0.5).reshape(1, 1, hq, d)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= (1e-5 if dtype == torch.float32 else TOL)


@pytest.mark.parametrize("n,split", [(1000, 64), (1000, None), (2048, None), (2049, None), (10240, None)])
def test_interleaved_partials_cover_round_robin_tiles(gpu, n, split):
    """tc_decode_partial_interleaved: split s's partial is the softmax over the 16-token tiles
    s*W + w + j*W*S (w < W) of its head, W = 2 waves for a cache of at most TC_DECODE_SHORT_TOKENS
    tokens and 4 above, in float64 within 1e-4; partial + combine is bit-identical to
    tc_decode_attention (the same kernels and plan)."""
    q, k, v, _ = workloads.decode_inputs(43, n=n)
    hkv, g, d = 8, 4, 128
    qd = q.to(gpu).reshape(1, hkv, g, d)
    kd, vd = k.to(gpu), v.to(gpu)
    S = flash_decode.num_splits(1, hkv, n, split)
    T = flash_decode.split_tokens(1, hkv, n, split)
    print(f"case: interleaved partials n={n} S={S} T={T}", flush=True)
    o = torch.empty((1, hkv, S, g, d), dtype=torch.float32, device=gpu)
    lse = torch.empty((1, hkv, S, g), dtype=torch.float32, device=gpu)
    lib = _lib.load()
    st = lambda t: _lib.i64x3(*[t.stride(i) if t.shape[i] > 1 else 0 for i in range(3)])
    rc = lib.tc_decode_partial_interleaved(qd.data_ptr(), st(qd), kd.data_ptr(), st(kd), vd.data_ptr(), st(vd),
                                           None, n, 1, hkv, g, d, _lib.TC_DTYPE_F16, SCALE, T, S, o.data_ptr(),
                                           lse.data_ptr(), _lib.stream_of(gpu))
    _lib.check(rc, "tc_decode_partial_interleaved")
    out = torch.empty_like(qd)
    rc = lib.tc_decode_combine(o.data_ptr(), lse.data_ptr(), 1, hkv, g, d, S, out.data_ptr(), st(out),
                               _lib.TC_DTYPE_F16, _lib.stream_of(gpu))
    _lib.check(rc, "tc_decode_combine")
    ref = flash_decode.decode_attention_batched(qd, kd, vd, SCALE, split=split)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    qn, kn, vn = q.float().numpy().reshape(hkv, g, d).astype(np.float64), k[0].float().numpy(), v[0].float().numpy()
    tiles = np.arange(-(-n // 16))
    W = 2 if n <= _lib.TC_DECODE_SHORT_TOKENS else 4
    for s in range(S):
        mine = tiles[(tiles // W) % S == s]
        toks = (mine[:, None] * 16 + np.arange(16)[None]).ravel()
        toks = toks[toks < n]
        if len(toks) == 0:
            assert bool(torch.isinf(lse[0, :, s]).all())
            continue
        sc = np.einsum("hgd,htd->hgt", qn, kn[:, toks].astype(np.float64)) * SCALE
        m = sc.max(-1, keepdims=True)
        p = np.exp(sc - m)
        want_o = np.einsum("hgt,htd->hgd", p / p.sum(-1, keepdims=True), vn[:, toks].astype(np.float64))
        want_l = (m[..., 0] + np.log(p.sum(-1)))
        assert np.abs(o[0, :, s].cpu().numpy() - want_o).max() <= 1e-4
        assert np.abs(lse[0, :, s].cpu().numpy() - want_l).max() <= 1e-4
