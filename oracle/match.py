"""Oracle of the request split — TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

``split`` restates threadcut/match.py:25-48 with plain Python loops (small
inputs only): A is the longest common prefix capped at len(new) - 1; every
start j > a whose min_suffix-token window equals new[a:a+min_suffix] is a
candidate, its run is lcp(cached[j:], new[a:]) capped at len(new[a:]) - 1,
and the first longest run wins.

Pins (tests/test_host.py): the reference's known answers
(tests/test_core.py:59-64) and an exhaustive search on random small inputs.
"""


def lcp(x, y):
    n = 0
    while n < min(len(x), len(y)) and x[n] == y[n]:
        n += 1
    return n


def split(cached, new, min_suffix=32, suffix=True):
    """(a, c0, c) of threadcut/match.py:33-48."""
    a = min(lcp(cached, new), len(new) - 1)
    rest = list(new[a:]) if a >= 0 else []
    if not suffix or len(rest) <= min_suffix or len(cached) - (a + 1) < min_suffix:
        return (a, a, 0)
    best = (a, a, 0)
    anchor = rest[:min_suffix]
    for j in range(a + 1, len(cached) - min_suffix + 1):
        if list(cached[j:j + min_suffix]) == anchor:
            c = min(lcp(cached[j:], rest), len(rest) - 1)
            if c > best[2]:
                best = (a, j, c)
    return best


def split_windows(cached, new, min_suffix=32, suffix=True):
    """threadcut/match.py:33-48 as the reference computes it: numpy sliding windows
    over cached[a+1:] compared with the anchor, then lcp per hit. Used to time the
    reference's CPU path next to the native matcher."""
    import numpy as np

    def np_lcp(x, y):
        n = min(len(x), len(y))
        if n == 0:
            return 0
        diff = np.flatnonzero(np.asarray(x[:n]) != np.asarray(y[:n]))
        return int(diff[0]) if len(diff) else n

    a = min(np_lcp(cached, new), len(new) - 1)
    rest = new[a:]
    if not suffix or len(rest) <= min_suffix or len(cached) - (a + 1) < min_suffix:
        return (a, a, 0)
    arr = np.asarray(cached)
    windows = np.lib.stride_tricks.sliding_window_view(arr[a + 1:], min_suffix)
    hits = np.flatnonzero((windows == np.asarray(rest[:min_suffix])).all(axis=1)) + a + 1
    best = (a, a, 0)
    for j in hits:
        c = min(np_lcp(cached[j:], rest), len(rest) - 1)
        if c > best[2]:
            best = (a, int(j), c)
    return best
