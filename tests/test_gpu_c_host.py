"""The HIP path driven from a plain C host program (tests/c_host/tc_host.c,
built with the library by threadcut_amd.build): device buffers from hipMalloc,
the C ABI's entry points, no Python or torch in that process, as a cgo / JNI /
N-API binding would drive it.

- Decode (tc_decode_attention with a hipMalloc workspace, and
  tc_decode_attention_noalloc): the golden fixtures against their float64
  outputs within 2e-3, and random fp16 / bf16 batches against the float64
  closed form of threadcut/flash_decode.py:57-69 (2e-3 fp16; bf16 4e-3 plus
  its half-ulp 2^-8 |x|). Both entry points bit-identical to each other and to
  the same call made through the Python wrapper in this process.
- Prefill (tc_prefill_attention, with tc_prefill_mask_tiles for a mask): g in
  1, 2, 4, 8, no mask, is_causal, broadcast and per-sequence boolean masks,
  against the float64 closed form of threadcut/attention.py:43-46 (2e-3 fp16,
  1.6e-2 bf16) and bit-identical to prefill.prefill_attention in this process.
- The paged cache (tc_page_prune, tc_page_tiles, tc_paged_rotate_keys,
  tc_decode_paged_attention) on one sequence in shuffled pages: the pools'
  kept rows bit-exact against the oracle's splice of the logical sequence,
  decode against the float64 closed form, both bit-identical to PagedKV in
  this process given the same page order.
- Splice (tc_splice_rope over L layers): the golden fixtures and random
  multi-layer overlapping, short-gap and disjoint moves, bit-exact against the
  oracle's restatement of threadcut/kv.py:83-92.
"""
import os
import subprocess

import numpy as np
import pytest
import torch

from oracle import decode as od
from oracle import prefill as opf
from oracle import splice as osp
from threadcut_amd import flash_decode, prefill
from threadcut_amd.paged import PagedKV
from threadcut_amd.match import Split

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "tests", "c_host", "tc_host")
GOLDEN = os.path.join(ROOT, "tests", "golden")
D = 128
DTYPE_CODE = {torch.float16: 0, torch.bfloat16: 1}


def run_host(mode, d):
    if not os.access(HOST, os.X_OK):
        pytest.fail("tests/c_host/tc_host is not built: run python -m threadcut_amd.build")
    print(f"case: tc_host {mode} {d}", flush=True)
    r = subprocess.run([HOST, mode, str(d)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, f"tc_host exited {r.returncode}: {r.stderr}"
    return r.stdout


def bits(t):
    """A 2-byte CPU tensor's raw bytes."""
    return t.contiguous().view(torch.int16).numpy().tobytes()


def from_bits(raw, shape, dtype):
    return torch.from_numpy(np.frombuffer(raw, dtype=np.int16).copy()).view(dtype).reshape(shape)


def host_decode(tmp, q, k, v, scale, split, dtype, lens=None):
    """q [B, Hkv, G, D], k/v [B, Hkv, N, D] CPU tensors (lens: int32 [B] or None) -> (out,
    out_noalloc) from the C host."""
    b, hkv, g, _ = q.shape
    n = k.shape[2]
    if lens is not None:
        (tmp / "lens.bin").write_bytes(lens.numpy().astype(np.int32).tobytes())
    (tmp / "q.bin").write_bytes(bits(q))
    (tmp / "k.bin").write_bytes(bits(k))
    (tmp / "v.bin").write_bytes(bits(v))
    (tmp / "meta.txt").write_text(f"{b} {hkv} {g} {n} {D} {scale!r} {split} {DTYPE_CODE[dtype]} "
                                  f"{int(lens is not None)}\n")
    run_host("decode", tmp)
    return (from_bits((tmp / "out.bin").read_bytes(), q.shape, dtype),
            from_bits((tmp / "out_noalloc.bin").read_bytes(), q.shape, dtype))


@pytest.mark.parametrize("name", ["decode_g4_n300.npz", "decode_g2_n77.npz"])
def test_c_host_decode_reproduces_fixture(gpu, tmp_path, name):
    f = np.load(os.path.join(GOLDEN, name))
    q, k, v = (torch.from_numpy(f[x])[None] for x in ("q", "k", "v"))
    scale = float(np.float32(f["scale"]))
    out, out_na = host_decode(tmp_path, q, k, v, scale, 256, torch.float16)
    assert np.abs(out[0].float().numpy() - f["out64"]).max() <= 2e-3
    assert torch.equal(out.view(torch.int16), out_na.view(torch.int16))
    py = flash_decode.decode_attention_batched(q.to(gpu), k.to(gpu), v.to(gpu), scale, split=256)
    assert torch.equal(py.cpu().view(torch.int16), out.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("b,hkv,g,n,split", [(1, 8, 4, 10240, 0), (2, 8, 4, 3000, 256), (3, 2, 8, 777, 64),
                                             (1, 4, 1, 1, 0), (2, 1, 5, 4097, 0)])
def test_c_host_decode_matches_closed_form(gpu, tmp_path, dtype, b, hkv, g, n, split):
    gen = torch.Generator().manual_seed(n + 7 * g)
    q = torch.randn(b, hkv, g, D, generator=gen).to(dtype)
    k = torch.randn(b, hkv, n, D, generator=gen).to(dtype)
    v = torch.randn(b, hkv, n, D, generator=gen).to(dtype)
    scale = D ** -0.5
    out, out_na = host_decode(tmp_path, q, k, v, scale, split, dtype)
    want = od.attention_f64(q.float().numpy(), k.float().numpy(), v.float().numpy(), scale)
    tol, rel = (2e-3, 0.0) if dtype == torch.float16 else (4e-3, 2.0 ** -8)
    assert (np.abs(out.float().numpy() - want) - (tol + rel * np.abs(want))).max() <= 0
    assert torch.equal(out.view(torch.int16), out_na.view(torch.int16))
    py = flash_decode.decode_attention_batched(q.to(gpu), k.to(gpu), v.to(gpu), scale, split=split or None)
    assert torch.equal(py.cpu().view(torch.int16), out.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_c_host_ragged_decode(gpu, tmp_path, dtype):
    """Per-sequence lengths (tc_decode_attention's lens, empty and 1-token sequences included)."""
    b, hkv, g, n = 6, 8, 4, 5000
    gen = torch.Generator().manual_seed(99)
    q = torch.randn(b, hkv, g, D, generator=gen).to(dtype)
    k = torch.randn(b, hkv, n, D, generator=gen).to(dtype)
    v = torch.randn(b, hkv, n, D, generator=gen).to(dtype)
    lens = torch.tensor([5000, 0, 1, 1234, 4097, 17], dtype=torch.int32)
    scale = D ** -0.5
    out, out_na = host_decode(tmp_path, q, k, v, scale, 0, dtype, lens)
    want = od.decode_ragged(q.float().numpy(), k.float().numpy(), v.float().numpy(), lens.numpy(), scale)
    tol, rel = (2e-3, 0.0) if dtype == torch.float16 else (4e-3, 2.0 ** -8)
    assert (np.abs(out.float().numpy() - want) - (tol + rel * np.abs(want))).max() <= 0
    assert torch.equal(out.view(torch.int16), out_na.view(torch.int16))
    py = flash_decode.decode_attention_batched(q.to(gpu), k.to(gpu), v.to(gpu), scale, lens=lens.to(gpu))
    assert torch.equal(py.cpu().view(torch.int16), out.view(torch.int16))


@pytest.mark.parametrize("b,hq,hkv,ql,n,mode,dtype", [
    (1, 32, 8, 300, 1000, "causal", torch.float16),
    (2, 8, 8, 64, 64, "none", torch.bfloat16),
    (2, 16, 2, 200, 700, "mask_per_sequence", torch.float16),
    (1, 8, 4, 129, 2100, "mask_broadcast", torch.bfloat16),
    (2, 32, 8, 512, 4096, "causal", torch.float16),
])
def test_c_host_prefill_matches_closed_form(gpu, tmp_path, b, hq, hkv, ql, n, mode, dtype):
    gen = torch.Generator().manual_seed(ql + n)
    q = torch.randn(b, hq, ql, D, generator=gen).to(dtype)
    k = torch.randn(b, hkv, n, D, generator=gen).to(dtype)
    v = torch.randn(b, hkv, n, D, generator=gen).to(dtype)
    scale = D ** -0.5
    mask = None
    if mode.startswith("mask"):
        mb = b if mode == "mask_per_sequence" else 1
        chunk = torch.arange(n)[None, :] <= torch.arange(ql)[:, None] + (n - ql)
        mask = (chunk & (torch.rand(mb, ql, n, generator=gen) < 0.8))[:, None]  # [mb, 1, Q, N]
        (tmp_path / "mask.bin").write_bytes(mask[:, 0].to(torch.uint8).numpy().tobytes())
    (tmp_path / "q.bin").write_bytes(bits(q))
    (tmp_path / "k.bin").write_bytes(bits(k))
    (tmp_path / "v.bin").write_bytes(bits(v))
    (tmp_path / "meta.txt").write_text(f"{b} {hq} {hkv} {ql} {n} {D} {scale!r} {int(mode == 'causal')} "
                                       f"{0 if mask is None else mask.shape[0]} {DTYPE_CODE[dtype]}\n")
    run_host("prefill", tmp_path)
    out = from_bits((tmp_path / "out.bin").read_bytes(), (b, ql, hq, D), dtype)
    want = opf.prefill_f64(q.float().numpy(), k.float().numpy(), v.float().numpy(), scale,
                           None if mask is None else mask.numpy(), mode == "causal")
    tol = 2e-3 if dtype == torch.float16 else 1.6e-2
    assert np.abs(out.float().numpy() - want).max() <= tol
    py = prefill.prefill_attention(q.to(gpu), k.to(gpu), v.to(gpu), None if mask is None else mask.to(gpu), scale,
                                   mode == "causal")
    assert torch.equal(py.cpu().view(torch.int16), out.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hkv,g,n,pt,s", [
    (8, 4, 1000, 64, Split(100, 400, 600)),
    (2, 8, 333, 16, Split(10, 17, 300)),
    (4, 1, 129, 32, None),
    (1, 5, 2048, 32, Split(0, 2000, 48)),
    (2, 2, 700, 64, Split(650, 700, 0)),
])
def test_c_host_paged_prune_and_decode(gpu, tmp_path, dtype, hkv, g, n, pt, s):
    gen = torch.Generator().manual_seed(n + pt)
    q = torch.randn(1, hkv, g, D, generator=gen).to(dtype)
    k = torch.randn(hkv, n, D, generator=gen).to(dtype)
    v = torch.randn(hkv, n, D, generator=gen).to(dtype)
    pages = -(-n // pt) + 3
    order = torch.randperm(pages, generator=gen)
    scale = D ** -0.5
    inv = osp.default_inv_freq(1e6, D)
    a, c0, c = (n, n, 0) if s is None else (s.a, s.c0, s.c)
    cos, sin = osp.rope_table(-(c0 - a), inv)
    (tmp_path / "q.bin").write_bytes(bits(q))
    (tmp_path / "k.bin").write_bytes(bits(k))
    (tmp_path / "v.bin").write_bytes(bits(v))
    (tmp_path / "order.bin").write_bytes(order.numpy().astype(np.int64).tobytes())
    (tmp_path / "table.bin").write_bytes(np.concatenate((cos, sin)).astype(np.float32).tobytes())
    (tmp_path / "meta.txt").write_text(f"{hkv} {g} {n} {D} {scale!r} {pt} {pages} {a} {c0} {c} "
                                       f"{DTYPE_CODE[dtype]}\n")
    run_host("paged", tmp_path)
    out = from_bits((tmp_path / "out.bin").read_bytes(), q.shape, dtype)
    kp = from_bits((tmp_path / "k_pool.bin").read_bytes(), (pages, hkv, pt, D), dtype)
    vp = from_bits((tmp_path / "v_pool.bin").read_bytes(), (pages, hkv, pt, D), dtype)
    frags = np.frombuffer((tmp_path / "frags.bin").read_bytes(), dtype=np.int64).reshape(-1, 3)
    k_kept = torch.cat([kp[p, :, f:f + m] for p, f, m in frags], 1)
    v_kept = torch.cat([vp[p, :, f:f + m] for p, f, m in frags], 1)

    name = "float16" if dtype == torch.float16 else "bfloat16"
    as_np = (lambda t: t.numpy()) if dtype == torch.float16 else (lambda t: t.view(torch.int16).numpy().view(np.uint16))
    kw, vw = osp.splice_copy(as_np(k), as_np(v), a, c0, c, cos, sin, dtype=name)
    assert np.array_equal(as_np(k_kept).view(np.uint16), kw.view(np.uint16))
    assert np.array_equal(as_np(v_kept).view(np.uint16), vw.view(np.uint16))
    want = od.attention_f64(q.float().numpy(), k_kept[None].float().numpy(), v_kept[None].float().numpy(), scale)
    tol, rel = (2e-3, 0.0) if dtype == torch.float16 else (4e-3, 2.0 ** -8)
    assert (np.abs(out.float().numpy() - want) - (tol + rel * np.abs(want))).max() <= 0

    cache = PagedKV(1, hkv, pages, pt, batch=1, dtype=dtype, device=gpu)
    cache.table.free = order.flip(0).tolist()  # pop() hands the pages out in `order`
    cache.append(0, [k.to(gpu)], [v.to(gpu)])
    if s is not None:
        cache.prune(0, s, inv)
    py = cache.decode(0, q.to(gpu), scale)
    assert torch.equal(py.cpu().view(torch.int16), out.view(torch.int16))
    kg, vg = cache.gather(0)
    assert torch.equal(kg.cpu().view(torch.int16), k_kept.view(torch.int16))
    assert torch.equal(vg.cpu().view(torch.int16), v_kept.view(torch.int16))


def host_splice(tmp, ks, vs, s, cos, sin, dtype):
    """ks/vs [L, B, H, cap, D] CPU tensors -> spliced (ks, vs) from the C host."""
    layers, b, h, cap, _ = ks.shape
    (tmp / "k.bin").write_bytes(bits(ks))
    (tmp / "v.bin").write_bytes(bits(vs))
    (tmp / "table.bin").write_bytes(np.concatenate((cos, sin)).astype(np.float32).tobytes())
    (tmp / "meta.txt").write_text(f"{layers} {b} {h} {cap} {D} {s.a} {s.c0} {s.c} {DTYPE_CODE[dtype]}\n")
    run_host("splice", tmp)
    return (from_bits((tmp / "k_out.bin").read_bytes(), ks.shape, dtype),
            from_bits((tmp / "v_out.bin").read_bytes(), vs.shape, dtype))


@pytest.mark.parametrize("name", ["splice_overlap_n40.npz", "splice_gap_n96.npz"])
def test_c_host_splice_reproduces_fixture(gpu, tmp_path, name):
    f = np.load(os.path.join(GOLDEN, name))
    s = Split(*(int(x) for x in f["split"]))
    ks, vs = torch.from_numpy(f["k"])[None], torch.from_numpy(f["v"])[None]
    k_out, v_out = host_splice(tmp_path, ks, vs, s, f["cos"], f["sin"], torch.float16)
    assert np.array_equal(k_out[0].numpy().view(np.uint16), f["k_out"].view(np.uint16))
    assert np.array_equal(v_out[0].numpy().view(np.uint16), f["v_out"].view(np.uint16))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("layers,b,h,cap,s", [
    (3, 2, 4, 300, Split(37, 58, 200)),     # overlapping, gap 21: the strip walk
    (2, 1, 8, 700, Split(10, 150, 500)),    # overlapping, gap 140: chain walks
    (4, 1, 2, 400, Split(5, 250, 120)),     # disjoint
    (1, 1, 1, 64, Split(0, 1, 63)),         # gap 1 over the whole buffer
])
def test_c_host_splice_matches_oracle(gpu, tmp_path, dtype, layers, b, h, cap, s):
    gen = torch.Generator().manual_seed(cap + s.c0)
    ks = torch.randn(layers, b, h, cap, D, generator=gen).to(dtype)
    vs = torch.randn(layers, b, h, cap, D, generator=gen).to(dtype)
    inv = osp.default_inv_freq(1e6, D)
    cos, sin = osp.rope_table(-s.gap, inv)
    k_out, v_out = host_splice(tmp_path, ks, vs, s, cos, sin, dtype)
    name = "float16" if dtype == torch.float16 else "bfloat16"
    for l in range(layers):
        k_in = ks[l].view(torch.int16).numpy().view(np.uint16) if dtype == torch.bfloat16 else ks[l].numpy()
        v_in = vs[l].view(torch.int16).numpy().view(np.uint16) if dtype == torch.bfloat16 else vs[l].numpy()
        kw, vw, n = osp.splice_growing(k_in, v_in, cap, s.a, s.c0, s.c, cos, sin, dtype=name)
        assert n == s.a + s.c
        assert np.array_equal(k_out[l].view(torch.int16).numpy().view(np.uint16), kw.view(np.uint16))
        assert np.array_equal(v_out[l].view(torch.int16).numpy().view(np.uint16), vw.view(np.uint16))
