"""Every entry point enqueues on the caller's current stream.

On a side stream (default priority, non-blocking), a spin kernel holds the
stream for milliseconds, the inputs are then written on that stream by
device-to-device copies from sources already on the GPU, and the call
follows. A launch on any other stream would run at once and read
the inputs as they were before the writes (zeros, or the cache before it was
filled), so a wrong stream shows as a wrong result, not as a flaky one. Each
result is checked against the oracle: decode and fused-append decode (float64
closed form, 2e-3), prefill (float64 closed form, 2e-3), the GrowingLayer
splice (bit-exact) and the paged prune + decode.
"""
import numpy as np
import pytest
import torch

from oracle import decode as od
from oracle import prefill as opf
from oracle import splice as osp
from threadcut_amd import flash_decode, kv, prefill, workloads
from threadcut_amd.match import Split
from threadcut_amd.paged import PagedKV

pytestmark = pytest.mark.gpu

D = 128
SPIN = 100_000_000  # cycles of torch.cuda._sleep's counter: tens of milliseconds or more


def rnd(shape, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)).half()


def on_side_stream(gpu, fn):
    """Run fn() on a fresh side stream after a spin kernel; return its result once done.
    The stream must still be spinning when fn() has enqueued everything, or a launch on a
    wrong stream could have found its inputs ready."""
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        torch.cuda._sleep(SPIN)
        out = fn()
    assert not side.query(), "the spin ended before the calls were enqueued"
    side.synchronize()
    return out


def test_decode_and_fused_append_on_a_side_stream(gpu):
    b, hkv, g, n = 2, 8, 4, 3000
    qh, kh, vh = rnd((b, hkv, g, D), 1), rnd((b, hkv, n, D), 2), rnd((b, hkv, n, D), 3)
    qd, kd, vd = qh.to(gpu), kh.to(gpu), vh.to(gpu)
    q = torch.zeros_like(qd)
    kbuf = torch.zeros((b, hkv, n + 16, D), dtype=torch.float16, device=gpu)
    vbuf = torch.zeros_like(kbuf)

    def work():
        q.copy_(qd)
        kbuf[:, :, :n].copy_(kd)
        vbuf[:, :, :n].copy_(vd)
        plain = flash_decode.decode_attention_batched(q, kbuf[:, :, :n], vbuf[:, :, :n], D ** -0.5)
        out = torch.empty_like(q)
        # Append row n - 1 again from k_new / v_new (the same values) and attend n tokens.
        flash_decode.decode_append_into(q, kbuf, vbuf, kbuf[:, :, n - 1].clone(), vbuf[:, :, n - 1].clone(), n,
                                        D ** -0.5, out)
        return plain, out

    plain, fused = on_side_stream(gpu, work)
    want = od.attention_f64(qh.float().numpy(), kh.float().numpy(), vh.float().numpy(), D ** -0.5)
    assert np.abs(plain.float().cpu().numpy() - want).max() <= 2e-3
    assert np.abs(fused.float().cpu().numpy() - want).max() <= 2e-3


def test_prefill_on_a_side_stream(gpu):
    b, hq, hkv, ql, n = 1, 32, 8, 200, 900
    qh, kh, vh = rnd((b, hq, ql, D), 4), rnd((b, hkv, n, D), 5), rnd((b, hkv, n, D), 6)
    mh = (torch.arange(n)[None, :] <= torch.arange(ql)[:, None] + (n - ql))[None, None]
    srcs = [t.to(gpu) for t in (qh, kh, vh, mh)]
    q, k, v, m = (torch.zeros_like(t) for t in srcs)

    def work():
        for dst, src in zip((q, k, v, m), srcs):
            dst.copy_(src)
        return prefill.prefill_attention(q, k, v, m, D ** -0.5)

    out = on_side_stream(gpu, work)
    want = opf.prefill_f64(qh.float().numpy(), kh.float().numpy(), vh.float().numpy(), D ** -0.5, mh.numpy())
    assert np.abs(out.float().cpu().numpy() - want).max() <= 2e-3


def test_splice_on_a_side_stream(gpu):
    n, s = 600, Split(50, 80, 500)
    inv = workloads.inv_freq()
    kh, vh = rnd((1, 8, n, D), 7), rnd((1, 8, n, D), 8)
    kd, vd = kh.to(gpu), vh.to(gpu)
    layer = kv.GrowingLayer()
    layer.update(torch.zeros_like(kd), torch.zeros_like(vd))

    def work():
        layer.kbuf[:, :, :n].copy_(kd)
        layer.vbuf[:, :, :n].copy_(vd)
        layer.splice(s, inv)
        return layer.kbuf[:, :, :n].clone(), layer.vbuf[:, :, :n].clone()

    k_out, v_out = on_side_stream(gpu, work)
    cos, sin = osp.rope_table(-s.gap, inv)
    kw, vw, _ = osp.splice_growing(kh.numpy(), vh.numpy(), n, s.a, s.c0, s.c, cos, sin)
    assert np.array_equal(k_out.cpu().numpy().view(np.uint16), kw.view(np.uint16))
    assert np.array_equal(v_out.cpu().numpy().view(np.uint16), vw.view(np.uint16))


def test_paged_prune_and_decode_on_a_side_stream(gpu):
    n, s = 700, Split(100, 260, 440)
    inv = workloads.inv_freq()
    kh, vh, qh = rnd((8, n, D), 9), rnd((8, n, D), 10), rnd((1, 8, 4, D), 11)
    cache = PagedKV(1, 8, 64, 16, batch=1, device=gpu)
    srcs = [t.to(gpu) for t in (kh, vh, qh)]
    k, v, q = (torch.zeros_like(t) for t in srcs)

    def work():
        for dst, src in zip((k, v, q), srcs):
            dst.copy_(src)
        cache.append(0, [k], [v])
        cache.prune(0, s, inv)
        kg, vg = cache.gather(0)
        return cache.decode(0, q, D ** -0.5), kg, vg

    out, kg, vg = on_side_stream(gpu, work)
    cos, sin = osp.rope_table(-s.gap, inv)
    kw, vw = osp.splice_copy(kh.numpy(), vh.numpy(), s.a, s.c0, s.c, cos, sin)
    assert np.array_equal(kg.cpu().numpy().view(np.uint16), kw.view(np.uint16))
    assert np.array_equal(vg.cpu().numpy().view(np.uint16), vw.view(np.uint16))
    want = od.attention_f64(qh.float().numpy(), kw[None].astype(np.float32), vw[None].astype(np.float32), D ** -0.5)
    assert np.abs(out.float().cpu().numpy() - want).max() <= 2e-3
