"""Prefill parity on the GPU: the GQA-native HIP kernel vs the float64 oracle of
threadcut/attention.py:43-47 and vs the reference's own GPU route (repeat_kv +
torch SDPA) on the same seeded inputs.

Tolerance: max-abs 2e-3 for fp16 (the north-star attention bar); bf16 outputs
round to 8 bits, so bf16 gets 1.6e-2, and in every case the kernel's error
against float64 must not exceed 1.5x that of torch SDPA on the expanded K/V.
"""
import numpy as np
import pytest
import torch
from transformers.masking_utils import sdpa_mask

from oracle import prefill as op
from threadcut_amd import _lib, attention, prefill, workloads

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}
SCALE = 128 ** -0.5


def ref64(q, k, v, mask=None, causal=False, scale=SCALE):
    m = None if mask is None else mask.cpu().numpy()
    return op.prefill_f64(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(), scale,
                          mask=m, causal=causal)


def torch_route(q, k, v, mask, causal, scale=SCALE):
    """The reference's prefill on the GPU: expanded K/V and SDPA in the input dtype."""
    g = q.shape[1] // k.shape[1]
    out = torch.nn.functional.scaled_dot_product_attention(
        q, attention.repeat_kv(k, g), attention.repeat_kv(v, g), attn_mask=mask, scale=scale, is_causal=causal)
    return out.transpose(1, 2)


def check(q, k, v, mask=None, causal=False, scale=SCALE, label="", splits=None):
    print(f"case: {label} q={tuple(q.shape)} k={tuple(k.shape)} dtype={q.dtype} causal={causal} "
          f"mask={None if mask is None else tuple(mask.shape)} splits={splits}", flush=True)
    out = prefill.prefill_attention(q, k, v, mask, scale, causal, splits=splits)
    torch.cuda.synchronize()
    assert out.shape == (q.shape[0], q.shape[2], q.shape[1], q.shape[3]) and out.is_contiguous()
    want = ref64(q, k, v, mask, causal, scale)
    err = np.abs(out.float().cpu().numpy() - want).max()
    tref = torch_route(q, k, v, mask, causal, scale)
    terr = np.abs(tref.float().cpu().numpy() - want).max()
    assert err <= max(TOL[q.dtype], 1.5 * terr), (err, terr)
    return out


@pytest.mark.parametrize("g", [1, 2, 4, 8])
@pytest.mark.parametrize("n", [2, 3, 16, 17, 63, 64, 65, 130, 300])
def test_causal_full_prompt(gpu, g, n):
    """q == n, no mask: SDPA's is_causal."""
    q_heads, kv_heads = {1: (8, 8), 2: (16, 8), 4: (32, 8), 8: (16, 2)}[g]
    q, k, v = workloads.prefill_inputs(10 * g + n, q_len=n, n=n, q_heads=q_heads, kv_heads=kv_heads, device=gpu)
    check(q, k, v, causal=True, label=f"causal g={g}")


@pytest.mark.parametrize("q_len,past", [(1, 5), (2, 1), (5, 60), (37, 100), (64, 64), (65, 200), (300, 1000)])
def test_chunk_on_top_of_a_cache(gpu, q_len, past):
    """The engine's chunked prefill: the boolean mask sdpa_mask builds for queries at past.."""
    n = past + q_len
    q, k, v = workloads.prefill_inputs(q_len + past, q_len=q_len, n=n, device=gpu)
    mask = sdpa_mask(batch_size=1, q_length=q_len, kv_length=n, q_offset=past, device=gpu)
    if mask is None:  # q_len == 1 without padding: every key visible
        mask = torch.ones((1, 1, q_len, n), dtype=torch.bool, device=gpu)
    assert torch.equal(mask.cpu(), workloads.causal_mask(q_len, n))
    check(q, k, v, mask=mask, label="chunk")


@pytest.mark.parametrize("q_len,n", [(2, 2), (7, 50), (100, 333)])
def test_no_mask_attends_to_everything(gpu, q_len, n):
    q, k, v = workloads.prefill_inputs(q_len * n, q_len=q_len, n=n, device=gpu)
    check(q, k, v, label="full")


@pytest.mark.parametrize("batch_mask", [1, 3])
def test_random_masks_and_batches(gpu, batch_mask):
    b, L, n = 3, 70, 150
    q, k, v = workloads.prefill_inputs(5, batch=b, q_len=L, n=n, device=gpu)
    g = torch.Generator().manual_seed(batch_mask)
    m = torch.rand((batch_mask, 1, L, n), generator=g) < 0.3
    m[..., 7] = True
    check(q, k, v, mask=m.to(gpu), label=f"random mask batch {batch_mask}")


@pytest.mark.parametrize("offset,pitch", [(1, 264), (3, 267), (0, 261), (4, 264)])
def test_mask_views(gpu, offset, pitch):
    """Boolean masks that are views: a base 1 or 3 bytes into the allocation, or an odd row
    stride, leave the mask rows unaligned (bytes are read one by one); 4-aligned ones are
    read as words. Both against the float64 oracle."""
    L, n = 40, 257
    q, k, v = workloads.prefill_inputs(60 + offset, q_len=L, n=n, device=gpu)
    g = torch.Generator().manual_seed(pitch)
    big = (torch.rand((1, 1, L, pitch), generator=g) < 0.5).to(gpu)
    m = big[..., offset:offset + n]
    assert m.stride(-2) == pitch and not m.is_contiguous()
    check(q, k, v, mask=m, label=f"mask view offset {offset} pitch {pitch}")


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 16])
def test_key_splits(gpu, splits):
    """Splitting the keys across work-groups (LSE-merged) gives the same attention,
    for causal, masked-chunk and unmasked calls; more splits than tiles are clamped."""
    q, k, v = workloads.prefill_inputs(20 + splits, q_len=200, n=200, device=gpu)
    check(q, k, v, causal=True, splits=splits, label="split causal")
    q, k, v = workloads.prefill_inputs(30 + splits, q_len=70, n=900, device=gpu)
    check(q, k, v, mask=workloads.causal_mask(70, 900).to(gpu), splits=splits, label="split chunk")
    check(q, k, v, splits=splits, label="split full")
    g = torch.Generator().manual_seed(splits)
    m = torch.rand((1, 1, 70, 900), generator=g) < 0.05
    m[..., :3, :] = False  # rows with no visible key in any split
    out = check(q, k, v, mask=m.to(gpu), splits=splits, label="split sparse mask")
    assert torch.all(out[0, :3] == 0)


@pytest.mark.parametrize("splits", [2, 5])
def test_key_splits_with_batches(gpu, splits):
    """Key splits and the combine index batches correctly (per-batch mask, bf16 too)."""
    b, L, n = 3, 50, 700
    q, k, v = workloads.prefill_inputs(50 + splits, batch=b, q_len=L, n=n, device=gpu)
    g = torch.Generator().manual_seed(splits)
    m = torch.rand((b, 1, L, n), generator=g) < 0.4
    m[..., -1] = True
    check(q, k, v, mask=m.to(gpu), splits=splits, label="split batch mask")
    check(q, k, v, causal=False, splits=splits, label="split batch full")
    qb, kb, vb = (t.to(torch.bfloat16) for t in (q, k, v))
    check(qb, kb, vb, mask=workloads.causal_mask(L, n, batch=b).to(gpu), splits=splits, label="split batch bf16")


@pytest.mark.parametrize("splits", [1, 3])
def test_long_masked_map_row(gpu, splits):
    """A 40000-key mask (625 tiles) in one key range: a work-group holds the first 64
    words (512 tiles) of its tile-map row in registers and loads the rest. FULL, SKIP
    and MIXED runs cross that boundary; the split case starts ranges mid-row."""
    L, n = 40, 40000
    q, k, v = workloads.prefill_inputs(60 + splits, q_len=L, n=n, device=gpu)
    g = torch.Generator().manual_seed(splits)
    m = torch.zeros((1, 1, L, n), dtype=torch.bool)
    m[..., :5000] = True                                   # FULL tiles
    m[..., 30000:34000] = torch.rand((L, 4000), generator=g) < 0.3   # MIXED across tile 512
    m[..., 36000:36100] = True                             # FULL past the register words
    m[..., 39990:] = torch.rand((L, 10), generator=g) < 0.5  # the ragged last tile
    m[..., 7, :] = False                                   # a row that sees nothing
    out = check(q, k, v, mask=m.to(gpu), splits=splits, label=f"long map row splits={splits}")
    assert torch.all(out[0, 7] == 0)


def test_short_chunk_on_long_cache_uses_splits(gpu):
    """A few hundred new tokens on top of a 10k cache: too few query blocks to fill
    the GPU, so the keys are split."""
    s = prefill.num_splits(1, 300, 10000, 32, 8)
    assert s > 1
    # 10 query blocks x 8 heads, times the splits, still fit two work-groups per CU.
    assert 80 * s <= 2 * torch.cuda.get_device_properties(gpu).multi_processor_count
    assert prefill.num_splits(1, 2048, 9764, 32, 8) == 1
    # A chunk of half its keys or more (a prompt) runs unsplit; a short chunk on a longer cache splits.
    for q_len, n in ((256, 256), (512, 512), (1024, 1024), (1024, 2048)):
        assert prefill.num_splits(1, q_len, n, 32, 8) == 1, (q_len, n)
    assert prefill.num_splits(1, 512, 2560, 32, 8) > 1
    q, k, v = workloads.prefill_inputs(40, q_len=300, n=10000, device=gpu)
    check(q, k, v, mask=workloads.causal_mask(300, 10000).to(gpu), label="short chunk")


def classify_tiles(mask, q_heads, kv_heads):
    """The tile map by its definition, in numpy: per (mask batch, query block of 128/g
    tokens, 64-key tile): 0 no visible key, 1 all visible, 3 exactly the end-aligned
    causal rule, 2 otherwise."""
    m = mask[:, 0].cpu().numpy()
    mb, L, n = m.shape
    tokens = 128 // (q_heads // kv_heads)
    nblk, nt = -(-L // tokens), -(-n // 64)
    out = np.zeros((mb, nblk, nt), np.uint8)
    past = n - L
    for b in range(mb):
        for i in range(nblk):
            t0, t1 = i * tokens, min(L, (i + 1) * tokens)
            for j in range(nt):
                blk = np.zeros((t1 - t0, 64), bool)
                blk[:, :min(64, n - 64 * j)] = m[b, t0:t1, 64 * j:64 * j + 64]
                keys = 64 * j + np.arange(64)
                causal = (keys[None, :] <= past + np.arange(t0, t1)[:, None]) & (keys[None, :] < n)
                out[b, i, j] = 0 if not blk.any() else 1 if blk.all() else 3 if (blk == causal).all() else 2
    return out


def test_mask_tile_map(gpu):
    """The one-pass tile map equals the classification by definition (sdpa_mask's chunk
    mask, one flipped element, random masks per batch)."""
    cases = [workloads.causal_mask(200, 1000), workloads.causal_mask(37, 130, batch=2).clone()]
    cases[1][1, 0, 5, 3] = False  # batch 1 leaves the causal rule in one tile
    g = torch.Generator().manual_seed(3)
    cases.append(torch.rand((2, 1, 90, 300), generator=g) < 0.5)
    for m in cases:
        for hq, hkv in ((32, 8), (8, 8)):
            md = m.to(gpu)
            prefill._tile_cache = None
            tiles = prefill.mask_tiles(md, hq, hkv)
            torch.cuda.synchronize()
            want = classify_tiles(md if md.stride(0) else md[:1], hq, hkv)
            mb, nblk, nt = want.shape
            pitch = -(-nt // 8) * 8  # rows padded to 8 tiles, the padding SKIP (0)
            got = tiles.cpu().numpy()[:mb * nblk * pitch].reshape(mb, nblk, pitch)
            assert np.array_equal(got[..., :nt], want) and not got[..., nt:].any()
    assert 3 in classify_tiles(cases[0], 32, 8) and 2 in classify_tiles(cases[1], 32, 8)


def test_rows_without_visible_keys_are_zero(gpu):
    q, k, v = workloads.prefill_inputs(6, q_len=20, n=40, device=gpu)
    m = workloads.causal_mask(20, 40).clone()
    m[..., 5, :] = False
    m[..., 11, :] = False
    out = check(q, k, v, mask=m.to(gpu), label="empty rows")
    assert torch.all(out[0, 5] == 0) and torch.all(out[0, 11] == 0)


def test_bf16(gpu):
    q, k, v = workloads.prefill_inputs(8, q_len=150, n=400, dtype=torch.bfloat16, device=gpu)
    check(q, k, v, mask=workloads.causal_mask(150, 400).to(gpu), label="bf16 chunk")
    q, k, v = workloads.prefill_inputs(9, q_len=130, n=130, dtype=torch.bfloat16, device=gpu)
    check(q, k, v, causal=True, label="bf16 causal")


def test_strided_cache_views_and_scales(gpu):
    """K/V as views [.., :n, :] of larger buffers (the GrowingLayer layout), contiguous query, big scale."""
    q, k, v = workloads.prefill_inputs(11, q_len=90, n=90, device=gpu)
    kb = torch.zeros((1, 8, 256, 128), dtype=k.dtype, device=gpu)
    vb = torch.full((1, 8, 256, 128), float("nan"), dtype=k.dtype, device=gpu)
    kb[:, :, :90] = k
    vb[:, :, :90] = v
    check(q.contiguous(), kb[:, :, :90], vb[:, :, :90], causal=True, label="cache views")
    check(q, k, v, causal=True, scale=1.0, label="scale 1")
    check(q * 4, k, v, causal=True, scale=1.0, label="large scores")


def test_token_major_layouts(gpu):
    """K and/or V stored token-major ([B, N, H, D] seen as [B, H, N, D]: a 2 KB row pitch) and the
    two with different pitches, so the kernel's K and V rows come from different strides."""
    q, k, v = workloads.prefill_inputs(12, q_len=100, n=333, device=gpu)
    kt = k.transpose(1, 2).contiguous().transpose(1, 2)
    vt = v.transpose(1, 2).contiguous().transpose(1, 2)
    assert kt.stride(2) == 8 * 128 and kt.stride(1) == 128
    mask = workloads.causal_mask(100, 333).to(gpu)
    check(q, kt, vt, mask=mask, label="token-major K and V")
    check(q, k, vt, mask=mask, label="token-major V only")
    check(q, kt, v, causal=False, label="token-major K only, no mask")


def test_row_pitch_past_one_buffer_range(gpu):
    """K/V rows 10 MiB apart: n + 128 rows span more than 2^31 bytes, so the kernel cannot address a
    head's keys through one buffer range and takes a range per tile instead (the other tests, with
    ordinary pitches, take the one range). One KV head, g = 4, the chunk and the causal prompt."""
    n, q_len, pitch = 100, 36, 5 << 20  # elements between rows: (100 + 128) * 2 * pitch > 2^31 bytes
    assert (n + 128) * 2 * pitch >= 1 << 31
    q, k0, v0 = workloads.prefill_inputs(14, q_len=q_len, n=n, q_heads=4, kv_heads=1, device=gpu)
    rows = []
    for src in (k0, v0):
        store = torch.zeros((n - 1) * pitch + 128, dtype=src.dtype, device=gpu)
        view = store.as_strided((1, 1, n, 128), (n * pitch, n * pitch, pitch, 1))
        view.copy_(src)
        rows.append(view)
    k, v = rows
    assert k.stride(2) == pitch
    mask = workloads.causal_mask(q_len, n).to(gpu)
    check(q, k, v, mask=mask, label="10 MiB row pitch, chunk")
    qp, _, _ = workloads.prefill_inputs(15, q_len=n, n=n, q_heads=4, kv_heads=1, device=gpu)
    check(qp, k, v, causal=True, label="10 MiB row pitch, causal prompt")


def test_through_attention_interface(gpu, monkeypatch):
    """attention.attention() takes the kernel for both prefill masks the model produces: the
    reference's route (repeat_kv + SDPA, attention.py:43-46) raises if it is reached."""
    def no_sdpa(*args, **kwargs):
        raise AssertionError("a supported prefill call reached SDPA instead of the HIP kernel")

    monkeypatch.setattr(attention.F, "scaled_dot_product_attention", no_sdpa)
    monkeypatch.setattr(attention, "repeat_kv", no_sdpa)
    q, k, v = workloads.prefill_inputs(12, q_len=96, n=96, device=gpu)
    out, w = attention.attention(None, q, k, v, None, scaling=SCALE)
    assert w is None
    assert np.abs(out.float().cpu().numpy() - ref64(q, k, v, causal=True)).max() <= TOL[q.dtype]
    q, k, v = workloads.prefill_inputs(13, q_len=96, n=250, device=gpu)
    mask = sdpa_mask(batch_size=1, q_length=96, kv_length=250, q_offset=154, device=gpu)
    out, _ = attention.attention(None, q, k, v, mask, scaling=SCALE)
    assert np.abs(out.float().cpu().numpy() - ref64(q, k, v, mask)).max() <= TOL[q.dtype]


def test_workload_shape_vs_torch_route(gpu):
    """One 2048-token chunk on top of the 7716 tokens the splice keeps (32/8 heads): within
    tolerance of the reference's GPU route computed in fp32."""
    q, k, v = workloads.prefill_inputs(14, device=gpu)
    L, n = q.shape[2], k.shape[2]
    mask = workloads.causal_mask(L, n, device=gpu)
    print(f"case: workload chunk q={L} n={n}", flush=True)
    out = prefill.prefill_attention(q, k, v, mask, SCALE)
    outs = [torch_route(q[:, 8 * i:8 * i + 8].float(), k[:, 2 * i:2 * i + 2].float(),
                        v[:, 2 * i:2 * i + 2].float(), mask, False) for i in range(4)]
    ref = torch.cat(outs, 2)
    torch.cuda.synchronize()
    assert (out.float() - ref).abs().max().item() <= TOL[q.dtype]


def test_causal_prompt_at_full_grid(gpu):
    """A causal 2048-token prompt (32/8 heads): 512 work-groups, so long and short query
    blocks share CUs (the folded work order, with the causal longest-first order on top)."""
    q, k, v = workloads.prefill_inputs(15, q_len=2048, n=2048, device=gpu)
    print("case: causal prompt 2048", flush=True)
    out = prefill.prefill_attention(q, k, v, None, SCALE, True)
    outs = [torch_route(q[:, 8 * i:8 * i + 8].float(), k[:, 2 * i:2 * i + 2].float(),
                        v[:, 2 * i:2 * i + 2].float(), None, True) for i in range(4)]
    ref = torch.cat(outs, 2)
    torch.cuda.synchronize()
    assert (out.float() - ref).abs().max().item() <= TOL[q.dtype]


def test_rejects(gpu):
    q, k, v = workloads.prefill_inputs(15, q_len=8, n=8, q_heads=12, kv_heads=4, device=gpu)
    assert not prefill.supports(q, k, None)
    with pytest.raises(RuntimeError, match="group 3"):
        prefill.prefill_attention(q, k, v, None, SCALE, True)
    q, k, v = workloads.prefill_inputs(15, q_len=8, n=8, device=gpu)
    with pytest.raises(ValueError, match="either"):
        prefill.prefill_attention(q, k, v, workloads.causal_mask(8, 8).to(gpu), SCALE, True)
    with pytest.raises(ValueError, match="bool"):
        prefill.prefill_attention(q, k, v, torch.zeros((1, 1, 8, 8), device=gpu), SCALE)
    assert not prefill.supports(q, k, torch.zeros((1, 1, 8, 8), device=gpu))
    with pytest.raises(RuntimeError, match="q_len"):
        lib = _lib.load()
        rc = lib.tc_prefill_attention(q.data_ptr(), _lib.i64x3(0, 0, 0), k.data_ptr(), _lib.i64x3(0, 0, 128),
                                      v.data_ptr(), _lib.i64x3(0, 0, 128), None, None, None, 0, 1, 9, 8, 1, 32, 8,
                                      128, 0, SCALE, 1, None, 0, q.data_ptr(), _lib.i64x3(0, 0, 0), None)
        _lib.check(rc, "tc_prefill_attention")
