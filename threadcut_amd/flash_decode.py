"""Split-KV GQA decode attention (flash-decoding) on MI355X.

Drop-in for threadcut/flash_decode.py:57-69 (``decode_attention``). One decode
step has a single query token, so each KV head serves only g = Hq/Hkv query
rows. The partial kernel gives every (split, KV head, sequence) its own
256-thread work-group, streams that slice of K/V once from HBM with the g
query rows held in registers, and writes a partial output plus its
log-sum-exp; a second kernel merges the splits with softmax(lse) weights
(threadcut/flash_decode.py:68-69). Both are HIP kernels of
``libthreadcut_hip.so``; this module only checks tensors and passes pointers,
strides and the current stream.
"""
import functools

import torch

from . import _lib

HEAD_DIM = 128
SPLIT_GRANULE = 64  # tokens; split lengths are rounded up to this


def supports(query, key, value):
    """True if the HIP decode kernels take this attention-interface call:
    query [b, hq, 1, d], key/value [b, hkv, n, d] on one GPU, float16 or
    bfloat16, d = 128, 1 <= hq / hkv <= 8, contiguous last dimensions.
    Decided from the tensors alone, so a missing library still raises when a
    supported call reaches it."""
    b, hq, _, d = query.shape
    hkv = key.shape[1]
    if not (query.is_cuda and key.is_cuda and value.is_cuda):
        return False
    if not (query.device == key.device == value.device):
        return False
    if query.dtype not in _lib.DTYPES or key.dtype != query.dtype or value.dtype != query.dtype:
        return False
    if d != HEAD_DIM or hkv < 1 or hq % hkv or not 1 <= hq // hkv <= 8:
        return False
    return query.stride(-1) == 1 and key.stride(-1) == 1 and value.stride(-1) == 1


def num_splits(batch, kv_heads, n_tokens, split=None, ragged=False):
    """KV splits a call of this size uses (``split=None``: tuned to fill the GPU)."""
    lib = _lib.load()
    s = lib.tc_decode_num_splits(int(batch), int(kv_heads), int(n_tokens), int(split or 0), int(bool(ragged)))
    if s < 0:
        _lib.check(-s, "tc_decode_num_splits")
    return s


def split_tokens(batch, kv_heads, n_tokens, split=None, ragged=False):
    """Tokens per split a call of this size uses."""
    lib = _lib.load()
    t = lib.tc_decode_split_tokens(int(batch), int(kv_heads), int(n_tokens), int(split or 0), int(bool(ragged)))
    if t < 0:
        _lib.check(-t, "tc_decode_split_tokens")
    return t


def _check_qkv(q, k, v, what):
    _lib.require_gpu(q, k, v, what=what)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError(f"{what}: expected q [B,Hkv,G,D], k/v [B,Hkv,N,D]")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"{what}: q/k/v dtypes differ ({q.dtype}, {k.dtype}, {v.dtype})")
    if not (q.device == k.device == v.device):
        raise ValueError(f"{what}: q/k/v on different devices")
    b, hkv, g, d = q.shape
    if k.shape[:2] != (b, hkv) or v.shape[:2] != (b, hkv) or k.shape[3] != d or v.shape[3] != d:
        raise ValueError(f"{what}: shapes q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)} disagree")
    if v.shape[2] != k.shape[2]:
        raise ValueError(f"{what}: k and v hold {k.shape[2]} and {v.shape[2]} tokens")
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.stride(3) != 1:
            raise ValueError(f"{what}: {name} must have a contiguous last dimension")


def _strides3(t, token_dim=False):
    """Element strides of dims 0-2; size-1 dims get a harmless canonical stride."""
    st = [t.stride(i) if t.shape[i] > 1 else 0 for i in range(3)]
    if token_dim and t.shape[2] <= 1:
        st[2] = t.shape[3]
    return _lib.i64x3(*st)


@functools.lru_cache(maxsize=1024)
def _plan(device_index, b, hkv, g, d, n, split, ragged):
    """(splits, workspace bytes) of a call; the tuned plan depends on the device's compute units,
    so it is computed with that device current."""
    lib = _lib.load()
    with torch.cuda.device(device_index):
        s = num_splits(b, hkv, n, split, ragged)
    return s, max(lib.tc_decode_workspace_bytes(b, hkv, g, d, s), 16)


def _on_device(device):
    """Context that makes `device` current, or nothing when it already is (the common case)."""
    if device.index is None or device.index == torch.cuda.current_device():
        return _NO_SWITCH
    return torch.cuda.device(device)


class _NoSwitch:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_NO_SWITCH = _NoSwitch()


def decode_into(q, k, v, scale, out, lens=None, split=None):
    """out[b,h,g,:] = softmax(q[b,h,g]·k[b,h,:len_b]ᵀ·scale)·v[b,h,:len_b] (fp32 math).

    q [B,Hkv,G,D], k/v [B,Hkv,N,D] (any strides, last dim contiguous), out
    [B,Hkv,G,D] in q.dtype, lens optional int32 [B] on the device (every
    lens[b] <= N; without lens all N tokens are used). Enqueued on the
    current stream; returns out.
    """
    _check_qkv(q, k, v, "decode_attention")
    b, hkv, g, d = q.shape
    n = k.shape[2]
    if out.shape != q.shape or out.dtype != q.dtype or out.device != q.device or out.stride(3) != 1:
        raise ValueError("decode_attention: out must match q in shape, dtype and device")
    if lens is not None:
        if lens.dtype != torch.int32 or lens.device != q.device or lens.shape != (b,) or not lens.is_contiguous():
            raise ValueError("decode_attention: lens must be a contiguous int32 [B] tensor on the device")
    lib = _lib.load()
    dt = _lib.dtype_code(q.dtype)
    _, nbytes = _plan(q.device.index, b, hkv, g, d, n, split, lens is not None)
    with _on_device(q.device):
        ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
        rc = lib.tc_decode_attention(
            q.data_ptr(), _strides3(q), k.data_ptr(), _strides3(k, True), v.data_ptr(), _strides3(v, True),
            lens.data_ptr() if lens is not None else None, n,
            b, hkv, g, d, dt, float(scale), int(split or 0),
            ws.data_ptr(), ws.numel(), out.data_ptr(), _strides3(out), _lib.stream_of(q.device))
        _lib.check(rc, "tc_decode_attention")
    return out


def decode_append_into(q, k_cache, v_cache, k_new, v_new, n, scale, out, split=None):
    """One decode step with the cache append fused in.

    k_cache/v_cache [B,Hkv,cap,D] (cap >= n), k_new/v_new [B,Hkv,1,D] or
    [B,Hkv,D]: the new rows are written to token n - 1 of the caches and q
    attends over tokens [0, n). out [B,Hkv,G,D]. Enqueued on the current stream.
    """
    _check_qkv(q, k_cache, v_cache, "decode_append")
    b, hkv, g, d = q.shape
    kn = k_new.reshape(b, hkv, d) if k_new.dim() == 4 else k_new
    vn = v_new.reshape(b, hkv, d) if v_new.dim() == 4 else v_new
    _lib.require_gpu(kn, vn, out, what="decode_append")
    if kn.shape != (b, hkv, d) or vn.shape != (b, hkv, d) or kn.dtype != q.dtype or vn.dtype != q.dtype:
        raise ValueError("decode_append: new K/V must be [B, Hkv, D] in the query dtype")
    if kn.stride(2) != 1 or vn.stride(2) != 1:
        raise ValueError("decode_append: new K/V need a contiguous last dimension")
    if not 1 <= n <= k_cache.shape[2]:
        raise ValueError(f"decode_append: n={n} outside [1, {k_cache.shape[2]}]")
    if out.shape != q.shape or out.dtype != q.dtype or out.stride(3) != 1:
        raise ValueError("decode_append: out must match q")
    lib = _lib.load()
    _, nbytes = _plan(q.device.index, b, hkv, g, d, int(n), split, False)
    with _on_device(q.device):
        ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
        st2 = lambda t: _lib.i64x2(t.stride(0) if t.shape[0] > 1 else 0, t.stride(1) if t.shape[1] > 1 else 0)
        rc = lib.tc_decode_append_attention(
            q.data_ptr(), _strides3(q), k_cache.data_ptr(), _strides3(k_cache, True), v_cache.data_ptr(),
            _strides3(v_cache, True), kn.data_ptr(), st2(kn), vn.data_ptr(), st2(vn), int(n),
            b, hkv, g, d, _lib.dtype_code(q.dtype), float(scale), int(split or 0),
            ws.data_ptr(), ws.numel(), out.data_ptr(), _strides3(out), _lib.stream_of(q.device))
        _lib.check(rc, "tc_decode_append_attention")
    return out


def decode_append_at(q, k_cache, v_cache, k_new, v_new, pos, scale, out, split=None):
    """decode_append_into with the append position on the device (graph-capturable).

    pos: int32 [B] on the device, the number of tokens already cached per
    sequence: the new rows go to token pos[b] of k_cache/v_cache [B,Hkv,cap,D]
    and q attends over tokens [0, pos[b]]. Nothing here reads pos on the host,
    so a captured graph of this call stays valid while pos advances. The split
    plan depends on cap only.
    """
    _check_qkv(q, k_cache, v_cache, "decode_append_at")
    b, hkv, g, d = q.shape
    kn = k_new.reshape(b, hkv, d) if k_new.dim() == 4 else k_new
    vn = v_new.reshape(b, hkv, d) if v_new.dim() == 4 else v_new
    _lib.require_gpu(kn, vn, out, pos, what="decode_append_at")
    if kn.shape != (b, hkv, d) or vn.shape != (b, hkv, d) or kn.dtype != q.dtype or vn.dtype != q.dtype:
        raise ValueError("decode_append_at: new K/V must be [B, Hkv, D] in the query dtype")
    if kn.stride(2) != 1 or vn.stride(2) != 1:
        raise ValueError("decode_append_at: new K/V need a contiguous last dimension")
    if pos.dtype != torch.int32 or pos.shape != (b,) or not pos.is_contiguous() or pos.device != q.device:
        raise ValueError("decode_append_at: pos must be a contiguous int32 [B] tensor on the device")
    if out.shape != q.shape or out.dtype != q.dtype or out.stride(3) != 1:
        raise ValueError("decode_append_at: out must match q")
    cap = k_cache.shape[2]
    lib = _lib.load()
    _, nbytes = _plan(q.device.index, b, hkv, g, d, int(cap), split, False)
    with _on_device(q.device):
        ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
        st2 = lambda t: _lib.i64x2(t.stride(0) if t.shape[0] > 1 else 0, t.stride(1) if t.shape[1] > 1 else 0)
        rc = lib.tc_decode_append_attention_at(
            q.data_ptr(), _strides3(q), k_cache.data_ptr(), _strides3(k_cache, True), v_cache.data_ptr(),
            _strides3(v_cache, True), kn.data_ptr(), st2(kn), vn.data_ptr(), st2(vn), pos.data_ptr(), int(cap),
            b, hkv, g, d, _lib.dtype_code(q.dtype), float(scale), int(split or 0),
            ws.data_ptr(), ws.numel(), out.data_ptr(), _strides3(out), _lib.stream_of(q.device))
        _lib.check(rc, "tc_decode_append_attention_at")
    return out


def decode_attention_batched(q, k, v, scale, lens=None, split=None):
    """Batched form: q [B,Hkv,G,D], k/v [B,Hkv,N,D] → [B,Hkv,G,D] in q.dtype."""
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    return decode_into(q, k, v, scale, out, lens=lens, split=split)


def decode_attention(q, k, v, scale, split=None, block=16):
    """q: [hkv, g, d]; k, v: [hkv, n, d] (last dim contiguous). Returns [hkv, g, d].

    Signature of threadcut/flash_decode.py:57. ``split`` is the number of
    tokens per KV split (rounded up to 64); None tunes it so the work-groups
    fill the GPU. ``block`` is accepted for compatibility: the kernel's
    token block is fixed at 16 per wave.
    """
    del block
    return decode_attention_batched(q[None], k[None], v[None], scale, split=split)[0]


class DecodePlan:
    """A decode call with fixed tensors, prepared once and launched many times.

    Holds the ctypes arguments and a workspace, so ``run()`` is one library
    call with no allocation (usable inside HIP graph capture). The tensors
    must stay alive and keep their storage while the plan is used.

    ``workspace`` (a uint8 device tensor of at least ``workspace_bytes``) lets
    plans that run one after another on one stream, such as the layers of a
    decode step, share one buffer: each call's partials are then written over
    the previous call's, whose lines are still in the L2 cache, and the
    combine reads them there (36 layers at 10240 tokens: 10.8 against 11.3 us
    a call with a buffer per layer). Plans sharing a workspace must not run
    concurrently.
    """

    def __init__(self, q, k, v, scale, out, lens=None, split=None, workspace=None):
        _check_qkv(q, k, v, "DecodePlan")
        b, hkv, g, d = q.shape
        self.lib = _lib.load()
        self.device = q.device
        with torch.cuda.device(q.device):
            ragged = lens is not None
            self.splits = num_splits(b, hkv, k.shape[2], split, ragged)
            self.split_tokens = split_tokens(b, hkv, k.shape[2], split, ragged)
            nbytes = self.lib.tc_decode_workspace_bytes(b, hkv, g, d, self.splits)
            self.workspace_bytes = max(nbytes, 16)
            if workspace is None:
                self.workspace = torch.empty(self.workspace_bytes, dtype=torch.uint8, device=q.device)
            else:
                if (workspace.dtype != torch.uint8 or workspace.device != q.device or not workspace.is_contiguous()
                        or workspace.numel() < self.workspace_bytes):
                    raise ValueError(f"DecodePlan: workspace must be a contiguous uint8 tensor on {q.device} "
                                     f"of at least {self.workspace_bytes} bytes")
                self.workspace = workspace
        self.tensors = (q, k, v, out, lens)
        self.args = (q.data_ptr(), _strides3(q), k.data_ptr(), _strides3(k, True), v.data_ptr(),
                     _strides3(v, True), lens.data_ptr() if lens is not None else None, k.shape[2],
                     b, hkv, g, d, _lib.dtype_code(q.dtype), float(scale), int(split or 0),
                     self.workspace.data_ptr(), self.workspace.numel(), out.data_ptr(), _strides3(out))
        n = k.shape[2]
        parts = b * hkv * self.splits * g
        self.o_part = self.workspace.data_ptr()
        self.lse_part = self.o_part + parts * d * 4
        self.partial_args = (q.data_ptr(), _strides3(q), k.data_ptr(), _strides3(k, True), v.data_ptr(),
                             _strides3(v, True), lens.data_ptr() if lens is not None else None, n,
                             b, hkv, g, d, _lib.dtype_code(q.dtype), float(scale), self.split_tokens,
                             self.splits, self.o_part, self.lse_part)
        self.combine_args = (self.o_part, self.lse_part, b, hkv, g, d, self.splits, out.data_ptr(),
                             _strides3(out), _lib.dtype_code(q.dtype))

    def run(self, stream=None):
        """Both kernels on `stream` (default: the current stream)."""
        s = stream if stream is not None else _lib.stream_of(self.device)
        _lib.check(self.lib.tc_decode_attention(*self.args, s), "tc_decode_attention")

    def run_partial(self, stream=None):
        """The partial pass alone, with the round-robin tile schedule ``run()`` uses."""
        s = stream if stream is not None else _lib.stream_of(self.device)
        _lib.check(self.lib.tc_decode_partial_interleaved(*self.partial_args, s), "tc_decode_partial_interleaved")

    def run_partial_contiguous(self, stream=None):
        """The partial pass with contiguous splits (the reference's slicing)."""
        s = stream if stream is not None else _lib.stream_of(self.device)
        _lib.check(self.lib.tc_decode_partial(*self.partial_args, s), "tc_decode_partial")

    def run_combine(self, stream=None):
        s = stream if stream is not None else _lib.stream_of(self.device)
        _lib.check(self.lib.tc_decode_combine(*self.combine_args, s), "tc_decode_combine")
