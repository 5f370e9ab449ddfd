"""ctypes binding of ``libthreadcut_hip.so`` (declared in include/threadcut_hip.h).

The library is built in-tree by ``threadcut_amd.build``. Loading it is the
only way to reach the kernels: there is no fallback, and a missing library
raises ``RuntimeError`` naming the build command.
"""
import contextlib
import ctypes
import functools
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libthreadcut_hip.so")

TC_OK = 0
TC_ERR_INVALID_ARGUMENT = 1
TC_ERR_UNSUPPORTED = 2
TC_ERR_ALIGNMENT = 3
TC_ERR_WORKSPACE = 4
TC_ERR_HIP = 5

TC_DTYPE_F16 = 0
TC_DTYPE_BF16 = 1
TC_MAX_SPLITS = 4096
TC_DECODE_SHORT_TOKENS = 2048  # caches up to this long: two-wave partial work-groups
TC_DECODE_SCRATCH_BYTES = 8 << 20  # static scratch of tc_decode_attention_noalloc, per GPU

_DTYPES = {torch.float16: TC_DTYPE_F16, torch.bfloat16: TC_DTYPE_BF16}
DTYPES = tuple(_DTYPES)  # element types the kernels take

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_S = ctypes.c_size_t
_I64P = ctypes.POINTER(ctypes.c_int64)
_PP = ctypes.POINTER(ctypes.c_void_p)
_FP = ctypes.POINTER(ctypes.c_float)

# name -> (restype, argtypes); every extern "C" symbol of the header.
SIGNATURES = {
    "tc_strerror": (ctypes.c_char_p, [_I]),
    "tc_last_error": (ctypes.c_char_p, []),
    "tc_abi_version": (_I, []),
    "tc_decode_num_splits": (_I, [_I, _I, _I64, _I, _I]),
    "tc_decode_split_tokens": (_I, [_I, _I, _I64, _I, _I]),
    "tc_decode_workspace_bytes": (_S, [_I, _I, _I, _I, _I]),
    "tc_decode_partial": (_I, [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64, _I, _I, _I, _I, _I, _F, _I, _I,
                               _P, _P, _P]),
    "tc_decode_partial_interleaved": (_I, [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64, _I, _I, _I, _I, _I, _F, _I,
                                           _I, _P, _P, _P]),
    "tc_decode_combine": (_I, [_P, _P, _I, _I, _I, _I, _I, _P, _I64P, _I, _P]),
    "tc_decode_attention": (_I, [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64, _I, _I, _I, _I, _I, _F, _I,
                                 _P, _S, _P, _I64P, _P]),
    "tc_decode_attention_noalloc": (_I, [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64, _I, _I, _I, _I, _I, _F, _I,
                                         _P, _I64P, _P]),
    "tc_decode_append_attention": (_I, [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I64, _I, _I, _I,
                                        _I, _I, _F, _I, _P, _S, _P, _I64P, _P]),
    "tc_decode_append_attention_at": (_I, [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _P, _I64, _I,
                                           _I, _I, _I, _I, _F, _I, _P, _S, _P, _I64P, _P]),
    "tc_decode_paged_attention": (_I, [_P, _I64P, _P, _P, _I64P, _I, _I, _P, _P, _I64, _I, _I, _I, _I, _I, _F, _I,
                                       _P, _S, _P, _I64P, _P]),
    "tc_decode_paged_append_attention": (_I, [_P, _I64P, _P, _P, _I64P, _I, _I, _P, _P, _I64, _P, _I64P, _P,
                                              _I64P, _I, _I, _I, _I, _I, _F, _I, _P, _S, _P, _I64P, _P]),
    "tc_decode_paged_append_attention_at": (_I, [_P, _I64P, _P, _P, _I64P, _I, _I, _P, _P, _I64, _P, _I64, _P,
                                                 _P, _I64P, _P, _I64P, _I, _I, _I, _I, _I, _F, _I, _P, _S, _P,
                                                 _I64P, _P]),
    "tc_shift_keys": (_I, [_P, _I64P, _P, _I64P, _I, _I, _I64, _I, _I, _FP, _P]),
    "tc_splice_rope": (_I, [_PP, _PP, _I, _I64P, _I, _I, _I64, _I, _I, _I64, _I64, _I64, _FP, _P]),
    "tc_splice_copy": (_I, [_PP, _PP, _I64P, _I64, _PP, _PP, _I64P, _I, _I, _I, _I, _I, _I64, _I64, _I64,
                            _FP, _P]),
    "tc_paged_rotate_keys": (_I, [_PP, _I, _I64P, _I, _I, _P, _I64, _I, _I, _I, _FP, _P]),
    "tc_prefill_attention": (_I, [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _P, _S, _I, _I64, _I64, _I, _I,
                                  _I, _I, _I, _F, _I, _P, _S, _P, _I64P, _P]),
    "tc_prefill_paged_attention": (_I, [_P, _I64P, _P, _P, _I64P, _I, _P, _I64, _P, _I64P, _P, _S, _I, _I64, _I64,
                                        _I, _I, _I, _I, _I, _F, _I, _P, _S, _P, _I64P, _P]),
    "tc_prefill_num_splits": (_I, [_I, _I64, _I64, _I, _I]),
    "tc_prefill_workspace_bytes": (_S, [_I, _I64, _I, _I]),
    "tc_prefill_tiles_bytes": (_S, [_I64, _I64, _I, _I, _I]),
    "tc_prefill_mask_tiles": (_I, [_P, _I64P, _I, _I64, _I64, _I, _I, _P, _S, _P]),
    "tc_match_split": (_I, [_I64P, _I64, _I64P, _I64, _I64, _I, _I64P]),
    "tc_page_tiles": (_I64, [_P, _I64, _I64, _I64, _P, _I64]),
    "tc_page_prune": (_I, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _I64P]),
    "tc_page_token_offsets": (_I64, [_P, _I64, _I64, _I64, _I64, _P, _I64]),
}

_lock = threading.Lock()
_lib = None


def load():
    """The loaded library (loaded once). Raises RuntimeError if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"threadcut_amd: {LIB_PATH} is missing; build it with `python -m threadcut_amd.build` "
                    "(or __graft_entry__.build()). There is no fallback path.")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def bind(path):
    """Load another build of the library (the same ABI, e.g. ``libthreadcut_stamps.so``) with the
    signatures set; it is not made the wrappers' library (see ``using``)."""
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


@contextlib.contextmanager
def using(lib):
    """Within the block the wrappers call `lib` (a library from ``bind``) instead of the
    default build; the default comes back on exit. For measurement runs in one thread."""
    global _lib
    saved = load()
    with _lock:
        _lib = lib
    try:
        yield lib
    finally:
        with _lock:
            _lib = saved


def check(rc, what):
    """Raise RuntimeError with the library's message unless rc == TC_OK."""
    if rc != TC_OK:
        lib = load()
        msg = lib.tc_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {lib.tc_strerror(rc).decode()} ({msg})")


def dtype_code(t):
    try:
        return _DTYPES[t]
    except KeyError:
        raise TypeError(f"threadcut_amd kernels take float16 or bfloat16 tensors, got {t}") from None


@functools.lru_cache(maxsize=4096)
def _i64x3(a, b, c):
    return (ctypes.c_int64 * 3)(a, b, c)


def i64x3(a, b, c):
    """A C int64[3] of (a, b, c). The arrays are shared between calls with the same values (the
    library only reads them), so a decode call does not build its stride arrays anew."""
    return _i64x3(int(a), int(b), int(c))


def i64x2(a, b):
    return (ctypes.c_int64 * 2)(int(a), int(b))


def ptr_array(ptrs):
    return (ctypes.c_void_p * max(1, len(ptrs)))(*[ctypes.c_void_p(int(p)) for p in ptrs])


def float_array(t):
    """Host fp32 array from a CPU float32 tensor (kept alive by the caller)."""
    t = t.detach().to("cpu", torch.float32).contiguous()
    return (ctypes.c_float * t.numel())(*t.tolist())


def stream_of(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_gpu(*tensors, what):
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(f"{what}: threadcut_amd runs on the GPU (HIP) only; got a {t.device} tensor")
