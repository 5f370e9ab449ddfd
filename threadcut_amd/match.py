"""Split of a new request against the cached token sequence.

Same contract as threadcut/match.py:14-48:

    cached = A · B · C · (stale tail)      new = A · C · D

A is the longest common prefix (capped so D keeps at least one token), B the
span the agent pruned, C the longest run of the new tokens after A that also
appears in the cache after A (found from a ``min_suffix``-token anchor), and D
the rest, the only part the model runs. ``Split(a, c0, c)`` feeds
``kv.splice``. Host-side integer work, unchanged in meaning.
"""
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
    """Split `new` against `cached` (threadcut/match.py:33-48)."""
    a = min(lcp(cached, new), len(new) - 1)
    rest = new[a:]
    no_reuse = Split(a, a, 0)
    if not suffix or len(rest) <= min_suffix or len(cached) - (a + 1) < min_suffix:
        return no_reuse
    hay = np.asarray(cached[a + 1:])
    anchor = np.asarray(rest[:min_suffix])
    n_starts = len(hay) - min_suffix + 1
    hit = np.ones(n_starts, dtype=bool)
    for i, tok in enumerate(anchor):  # anchor token i must sit at start + i
        hit &= hay[i:i + n_starts] == tok
    best = no_reuse
    for off in np.flatnonzero(hit):
        j = a + 1 + int(off)
        c = min(lcp(cached[j:], rest), len(rest) - 1)
        if c > best.c:
            best = Split(a, j, c)
    return best
