"""Split of a new request against the cached token sequence.

Same contract as threadcut/match.py:14-48:

    cached = A · B · C · (stale tail)      new = A · C · D

A is the longest common prefix (capped so D keeps at least one token), B the
span the agent pruned, C the longest run of the new tokens after A that also
appears in the cache after A (found from a ``min_suffix``-token anchor), and D
the rest, the only part the model runs. ``Split(a, c0, c)`` feeds
``kv.splice``. Host-side integer work, unchanged in meaning; the search runs
in the library's C++ matcher.
"""
import ctypes
from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Split:
    a: int   # len(A)
    c0: int  # C starts at cached[c0]; B = cached[a:c0]
    c: int   # len(C); D = new[a + c:]

    @property
    def gap(self):
        return self.c0 - self.a


def lcp(x, y):
    """Length of the longest common prefix of two token sequences."""
    n = min(len(x), len(y))
    if n == 0:
        return 0
    ne = np.asarray(x[:n]) != np.asarray(y[:n])
    first = int(np.argmax(ne))
    return first if ne[first] else n


def split(cached, new, min_suffix=32, suffix=True):
    """Split `new` against `cached` (threadcut/match.py:33-48).

    Runs the native matcher (``tc_match_split``: rolling-hash anchor search,
    linear in the cache length); token ids are taken as 64-bit integers.
    """
    from . import _lib

    c = np.ascontiguousarray(np.asarray(cached, dtype=np.int64).reshape(-1))
    n = np.ascontiguousarray(np.asarray(new, dtype=np.int64).reshape(-1))
    out = (ctypes.c_int64 * 3)()
    p64 = ctypes.POINTER(ctypes.c_int64)
    rc = _lib.load().tc_match_split(c.ctypes.data_as(p64), len(c), n.ctypes.data_as(p64), len(n),
                                    int(min_suffix), int(bool(suffix)), out)
    _lib.check(rc, "tc_match_split")
    return Split(int(out[0]), int(out[1]), int(out[2]))
