"""The C ABI without a GPU: the library loads, exports every symbol the header
declares, and rejects bad arguments before it touches the device."""
import ctypes
import os
import re

import pytest

from threadcut_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "threadcut_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const char\*|int|int64_t|size_t)\s+(tc_\w+)\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(_lib.SIGNATURES)


def test_every_declared_symbol_is_exported(lib):
    for name in declared_symbols():
        assert hasattr(lib, name), name
        assert ctypes.cast(getattr(lib, name), ctypes.c_void_p).value


def test_measurement_build_exports_the_abi_and_its_stamp_setters():
    """libthreadcut_stamps.so (the whole library built with the decode and prefill stamps)
    exports every declared symbol plus the two setters bench.py's timelines call."""
    from threadcut_amd import build
    stamps = _lib.bind(build.STAMPS_LIB)
    for name in declared_symbols() + ["tc_decode_set_stamps", "tc_prefill_set_stamps"]:
        assert hasattr(stamps, name), name
    # The wrappers call it inside `using` only.
    default = _lib.load()
    with _lib.using(stamps):
        assert _lib.load() is stamps
        assert _lib.load().tc_abi_version() == default.tc_abi_version()
    assert _lib.load() is default


def test_scratch_size_matches_header():
    m = re.search(r"#define TC_DECODE_SCRATCH_BYTES \((\d+)u << (\d+)\)", open(HEADER).read())
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.TC_DECODE_SCRATCH_BYTES


def test_short_cache_bound_matches_header():
    m = re.search(r"#define TC_DECODE_SHORT_TOKENS (\d+)", open(HEADER).read())
    assert m and int(m.group(1)) == _lib.TC_DECODE_SHORT_TOKENS


def test_noalloc_refuses_plans_beyond_its_scratch(lib):
    # 16 x 8 KV heads x 8 query heads at 64-token splits of 4096 tokens: 33 MB of partials.
    # Refused on the host (the split length is given, so no device is queried).
    b, h, g, d, n = 16, 8, 8, 128, 4096
    s = lib.tc_decode_num_splits(b, h, n, 64, 0)
    assert lib.tc_decode_workspace_bytes(b, h, g, d, s) > _lib.TC_DECODE_SCRATCH_BYTES
    st = _lib.i64x3(h * n * d, n * d, d)
    rc = lib.tc_decode_attention_noalloc(16, _lib.i64x3(h * g * d, g * d, d), 32, st, 48, st, None, n, b, h, g, d,
                                         _lib.TC_DTYPE_F16, 0.088, 64, 64, _lib.i64x3(h * g * d, g * d, d), None)
    assert rc == _lib.TC_ERR_WORKSPACE
    assert "static scratch" in lib.tc_last_error().decode()


def test_version_and_messages(lib):
    assert lib.tc_abi_version() == 2
    for code in range(6):
        assert lib.tc_strerror(code)
    assert lib.tc_strerror(99) == b"unknown error"


def test_split_arithmetic(lib):
    assert lib.tc_decode_split_tokens(1, 8, 10240, 256, 0) == 256
    assert lib.tc_decode_num_splits(1, 8, 10240, 256, 0) == 40      # cdiv(n, split) as the reference
    assert lib.tc_decode_split_tokens(1, 8, 10240, 100, 0) == 128   # rounded up to the 64-token granule
    assert lib.tc_decode_num_splits(1, 8, 10240, 100, 1) == 80
    assert lib.tc_decode_num_splits(1, 8, 0, 256, 0) == 0
    # Never more than TC_MAX_SPLITS splits: the split grows instead.
    n = 1 << 24
    assert lib.tc_decode_num_splits(1, 8, n, 64, 0) <= _lib.TC_MAX_SPLITS
    assert lib.tc_decode_split_tokens(1, 8, n, 64, 0) == n // _lib.TC_MAX_SPLITS
    assert lib.tc_decode_num_splits(0, 8, 100, 64, 0) == -_lib.TC_ERR_INVALID_ARGUMENT


def test_workspace_bytes(lib):
    b, h, g, d, s = 2, 8, 4, 128, 27
    assert lib.tc_decode_workspace_bytes(b, h, g, d, s) == b * h * s * g * (d + 1) * 4
    assert lib.tc_decode_workspace_bytes(b, h, g, d, 0) == 0


def _partial(lib, **kw):
    a = dict(q=16, qs=(4096, 512, 128), k=32, ks=(0, 1 << 20, 128), v=48, vs=(0, 1 << 20, 128), lens=None,
             n=1000, b=1, h=8, g=4, d=128, dt=0, scale=0.088, split=256, S=4, o=64, l=80)
    a.update(kw)
    return lib.tc_decode_partial(a["q"], _lib.i64x3(*a["qs"]), a["k"], _lib.i64x3(*a["ks"]), a["v"],
                                 _lib.i64x3(*a["vs"]), a["lens"], a["n"], a["b"], a["h"], a["g"], a["d"], a["dt"],
                                 a["scale"], a["split"], a["S"], a["o"], a["l"], None)


def test_decode_validation_before_any_device_call(lib):
    assert _partial(lib, d=96) == _lib.TC_ERR_UNSUPPORTED
    assert b"head_dim" in lib.tc_last_error()
    assert _partial(lib, g=9) == _lib.TC_ERR_UNSUPPORTED
    assert _partial(lib, dt=7) == _lib.TC_ERR_UNSUPPORTED
    assert _partial(lib, k=0) == _lib.TC_ERR_INVALID_ARGUMENT
    assert _partial(lib, q=17) == _lib.TC_ERR_ALIGNMENT
    assert _partial(lib, ks=(0, 1 << 20, 130)) == _lib.TC_ERR_ALIGNMENT
    assert _partial(lib, split=100) == _lib.TC_ERR_INVALID_ARGUMENT
    assert _partial(lib, S=3) == _lib.TC_ERR_INVALID_ARGUMENT            # 3 x 256 < 1000 tokens
    assert _partial(lib, S=_lib.TC_MAX_SPLITS + 1, split=64) == _lib.TC_ERR_INVALID_ARGUMENT
    assert _partial(lib, scale=float("inf")) == _lib.TC_ERR_INVALID_ARGUMENT
    assert _partial(lib, ks=(0, 1 << 20, 8)) == _lib.TC_ERR_INVALID_ARGUMENT  # rows would overlap
    # An empty cache needs no pointers and enqueues nothing.
    assert _partial(lib, n=0, S=0, k=0, v=0) == _lib.TC_OK


def test_combine_and_attention_validation(lib):
    rc = lib.tc_decode_combine(64, 80, 1, 8, 4, 64, 4, 16, _lib.i64x3(4096, 512, 128), 0, None)
    assert rc == _lib.TC_ERR_UNSUPPORTED
    rc = lib.tc_decode_combine(64, 80, 1, 8, 4, 128, 4, 0, _lib.i64x3(4096, 512, 128), 0, None)
    assert rc == _lib.TC_ERR_INVALID_ARGUMENT
    # A too-small workspace is reported (split length given, so no device query happens).
    rc = lib.tc_decode_attention(16, _lib.i64x3(4096, 512, 128), 32, _lib.i64x3(0, 1 << 20, 128), 48,
                                 _lib.i64x3(0, 1 << 20, 128), None, 1000, 1, 8, 4, 128, 0, 0.088, 256,
                                 64, 100, 16, _lib.i64x3(4096, 512, 128), None)
    assert rc == _lib.TC_ERR_WORKSPACE


def test_prefill_validation_before_any_device_call(lib):
    st = _lib.i64x3(1 << 24, 1 << 20, 128)

    def prefill(q_len=16, n=64, hq=32, hkv=8, d=128, dt=0, q=4096, causal=1):
        return lib.tc_prefill_attention(q, st, 8192, st, 12288, st, None, None, None, 0, causal, q_len, n, 1, hq, hkv,
                                        d, dt, 0.088, 0, None, 0, 16384, st, None)

    assert prefill(d=64) == _lib.TC_ERR_UNSUPPORTED
    assert prefill(hq=24) == _lib.TC_ERR_UNSUPPORTED                   # group 3
    assert prefill(q_len=65) == _lib.TC_ERR_INVALID_ARGUMENT           # more queries than keys
    assert prefill(q=4100) == _lib.TC_ERR_ALIGNMENT
    # Key positions are 32-bit in the kernel: 2^30 keys or more are refused.
    assert prefill(n=1 << 30) == _lib.TC_ERR_UNSUPPORTED
    assert b"2^30" in lib.tc_last_error()
    assert prefill(q_len=0, n=1 << 30) == _lib.TC_OK                   # nothing to do


def test_splice_validation(lib):
    ptrs = _lib.ptr_array([4096, 8192])
    st = _lib.i64x3(0, 1 << 20, 128)
    table = (ctypes.c_float * 128)()

    def splice(a, c0, c, kp=ptrs, cap=1000, s=st):
        return lib.tc_splice_rope(kp, ptrs, 2, s, 1, 8, cap, 128, 0, a, c0, c, table, None)

    assert splice(10, 5, 3) == _lib.TC_ERR_INVALID_ARGUMENT          # c0 < a
    assert splice(10, 990, 20) == _lib.TC_ERR_INVALID_ARGUMENT       # past the capacity
    assert splice(10, 20, 5, kp=_lib.ptr_array([4096, 0])) == _lib.TC_ERR_INVALID_ARGUMENT
    assert splice(10, 20, 5, kp=_lib.ptr_array([4096, 8200])) == _lib.TC_ERR_ALIGNMENT
    assert splice(10, 20, 5, s=_lib.i64x3(0, 1 << 20, 100)) == _lib.TC_ERR_ALIGNMENT
    # No gap or no suffix: nothing to move, nothing enqueued.
    assert splice(10, 10, 50) == _lib.TC_OK
    assert splice(10, 30, 0) == _lib.TC_OK
    # A copy that keeps nothing (a = c = 0) needs no pointers: the new cache is empty.
    rc = lib.tc_splice_copy(_lib.ptr_array([0]), _lib.ptr_array([0]), st, 5, _lib.ptr_array([0]),
                            _lib.ptr_array([0]), st, 1, 1, 8, 128, 0, 0, 5, 0, None, None)
    assert rc == _lib.TC_OK
    rc = lib.tc_splice_copy(_lib.ptr_array([0]), _lib.ptr_array([0]), st, 5, _lib.ptr_array([0]),
                            _lib.ptr_array([0]), st, 1, 1, 8, 128, 0, 1, 5, 0, None, None)
    assert rc == _lib.TC_ERR_INVALID_ARGUMENT  # one kept row needs its pointers
    rc = lib.tc_shift_keys(4096, st, 4096, st, 1, 8, 10, 128, 0, table, None)
    assert rc == _lib.TC_ERR_INVALID_ARGUMENT and b"alias" in lib.tc_last_error()
    assert lib.tc_shift_keys(4096, st, 8192, st, 1, 8, 0, 128, 0, table, None) == _lib.TC_OK


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(RuntimeError, match="no fallback"):
        _lib.load()
