"""The allocation-free decode entry point (tc_decode_attention_noalloc) through the C ABI.

It runs the kernels of tc_decode_attention with the split partials in the
library's static scratch array instead of a caller workspace, so its output
must equal that entry point's bit for bit on the same inputs and plan, and
stay within the decode bar (max-abs 2e-3, fp16) of the float64 closed form.
Two calls in a row, the second smaller, check that a call does not depend on
what the previous one left in the shared array.
"""
import numpy as np
import pytest
import torch

from oracle import decode as od
from threadcut_amd import _lib, flash_decode, workloads

pytestmark = pytest.mark.gpu

TOL = 2e-3
SCALE = 128 ** -0.5


def _strides(t):
    return _lib.i64x3(*[t.stride(i) if t.shape[i] > 1 else 0 for i in range(3)])


def _kv_strides(t):
    st = [t.stride(i) if t.shape[i] > 1 else 0 for i in range(3)]
    if t.shape[2] <= 1:
        st[2] = t.shape[3]
    return _lib.i64x3(*st)


def _both(dev, seed, batch, n, lens=None, dtype=torch.float16):
    """(noalloc output, workspace-entry output, float64 reference) for one seeded call."""
    q, k, v, _ = workloads.decode_inputs(seed, batch=batch, n=n, dtype=dtype)
    b, hq, _, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    qd = q.to(dev).reshape(b, hkv, g, d)
    kd, vd = k.to(dev), v.to(dev)
    ld = None if lens is None else lens.to(dev)
    lib = _lib.load()
    dt = _lib.dtype_code(dtype)
    stream = _lib.stream_of(dev)
    out_na = torch.full_like(qd, float("nan"))
    out_ws = torch.full_like(qd, float("nan"))
    with torch.cuda.device(dev):
        rc = lib.tc_decode_attention_noalloc(qd.data_ptr(), _strides(qd), kd.data_ptr(), _kv_strides(kd),
                                             vd.data_ptr(), _kv_strides(vd), None if ld is None else ld.data_ptr(),
                                             n, b, hkv, g, d, dt, SCALE, 0, out_na.data_ptr(), _strides(out_na),
                                             stream)
        _lib.check(rc, "tc_decode_attention_noalloc")
        s = flash_decode.num_splits(b, hkv, n, None, ragged=ld is not None)
        ws = torch.empty(max(lib.tc_decode_workspace_bytes(b, hkv, g, d, s), 16), dtype=torch.uint8, device=dev)
        rc = lib.tc_decode_attention(qd.data_ptr(), _strides(qd), kd.data_ptr(), _kv_strides(kd), vd.data_ptr(),
                                     _kv_strides(vd), None if ld is None else ld.data_ptr(), n, b, hkv, g, d, dt,
                                     SCALE, 0, ws.data_ptr(), ws.numel(), out_ws.data_ptr(), _strides(out_ws), stream)
        _lib.check(rc, "tc_decode_attention")
    torch.cuda.synchronize()
    qn = q.float().numpy().reshape(b, hkv, g, d)
    if lens is None:
        ref = od.attention_f64(qn, k.float().numpy(), v.float().numpy(), SCALE)
    else:
        ref = od.decode_ragged(qn, k.float().numpy(), v.float().numpy(), lens.numpy(), SCALE)
    return out_na.cpu(), out_ws.cpu(), ref


def test_noalloc_matches_workspace_entry_two_calls(gpu):
    """The 10240-token call of the decode sweep, then a smaller 1536-token call."""
    for seed, n in ((2, 10240), (0, 1536)):
        print(f"case: noalloc B=1 Hq=32 Hkv=8 n={n} seed {seed}", flush=True)
        na, ws, ref = _both(gpu, seed, 1, n)
        assert torch.equal(na, ws), f"n={n}: noalloc and workspace outputs differ"
        assert np.abs(na.float().numpy() - ref).max() <= TOL


def test_noalloc_ragged_then_single(gpu):
    """A ragged batch of 4 (per-sequence lengths), then a single short sequence in bf16."""
    lens = torch.tensor([4096, 17, 2500, 1], dtype=torch.int32)
    print("case: noalloc ragged B=4 n=4096 lens [4096, 17, 2500, 1]", flush=True)
    na, ws, ref = _both(gpu, 31, 4, 4096, lens=lens)
    assert torch.equal(na, ws)
    assert np.abs(na.float().numpy() - ref).max() <= TOL
    print("case: noalloc B=1 n=300 bf16", flush=True)
    na, ws, ref = _both(gpu, 32, 1, 300, dtype=torch.bfloat16)
    assert torch.equal(na, ws)
    assert np.abs(na.float().numpy() - ref).max() <= 4e-3


def test_noalloc_rejects_plans_beyond_the_scratch(gpu):
    """16 sequences x 8 KV heads x 8 query heads at 64-token splits of 4096 tokens need 33 MB of
    partials: refused on the host before anything is enqueued; the output keeps its contents."""
    b, hkv, g, d, n = 16, 8, 8, 128, 4096
    lib = _lib.load()
    s = lib.tc_decode_num_splits(b, hkv, n, 64, 0)
    assert lib.tc_decode_workspace_bytes(b, hkv, g, d, s) > _lib.TC_DECODE_SCRATCH_BYTES
    q = torch.zeros((b, hkv, g, d), dtype=torch.float16, device=gpu)
    k = torch.zeros((b, hkv, n, d), dtype=torch.float16, device=gpu)
    out = torch.full_like(q, 7.0)
    with torch.cuda.device(gpu):
        rc = lib.tc_decode_attention_noalloc(q.data_ptr(), _strides(q), k.data_ptr(), _kv_strides(k), k.data_ptr(),
                                             _kv_strides(k), None, n, b, hkv, g, d, _lib.TC_DTYPE_F16, SCALE, 64,
                                             out.data_ptr(), _strides(out), _lib.stream_of(gpu))
    assert rc == _lib.TC_ERR_WORKSPACE
    assert "static scratch" in lib.tc_last_error().decode()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
