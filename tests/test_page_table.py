"""The page-table arithmetic of the paged cache (tc_page_tiles, tc_page_prune,
tc_page_token_offsets; host code, no GPU) against a numpy restatement written
here from the definitions: a sequence is a list of fragments (page, first
slot, count) in logical order; its tiles cut every fragment at multiples of
16 slots; a prune keeps logical [0, a) and [c0, c0 + c) and frees the pages
nothing kept uses; a token's row sits page * page_bytes + slot * slot_bytes
into a head slab.
"""
import random

import numpy as np
import pytest

from threadcut_amd import _lib
from threadcut_amd.paged import PageTable, _tiles, tiles_of


def token_slots(frags):
    """(page, slot) of every token, by expanding each fragment."""
    out = [(p, s + j) for p, s, cnt in frags for j in range(cnt)]
    return np.array(out, dtype=np.int64).reshape(-1, 2)


def tiles_ref(frags, first_pos=0):
    out, pos = [], first_pos
    for p, s, cnt in frags:
        t = s // 16
        while t * 16 < s + cnt:
            lo, hi = max(s, t * 16), min(s + cnt, (t + 1) * 16)
            out.append((p, lo, hi - lo, pos))
            pos += hi - lo
            t += 1
    return np.array(out, dtype=np.int32).reshape(-1, 4)


def regroup(slots):
    """Fragments of a (page, slot) token list: runs of consecutive slots of one page."""
    frags = []
    for p, s in slots.tolist():
        if frags and frags[-1][0] == p and frags[-1][1] + frags[-1][2] == s:
            frags[-1][2] += 1
        else:
            frags.append([p, s, 1])
    return frags


def prune_ref(frags, a, c0, c):
    sl = token_slots(frags)
    kept_slots = np.concatenate([sl[:a], sl[c0:c0 + c]])
    suffix = regroup(sl[c0:c0 + c])
    kept = regroup(kept_slots)
    freed = sorted(set(int(x) for x in sl[:, 0]) - set(int(x) for x in kept_slots[:, 0]))
    return kept, suffix, freed


def random_frags(rnd, P, n_frags, pages):
    frags = []
    for _ in range(n_frags):
        s = rnd.randrange(P)
        frags.append([rnd.randrange(pages), s, rnd.randint(1, P - s)])
    return frags


def test_tiles_match_restatement():
    rnd = random.Random(0)
    for trial in range(300):
        P = rnd.choice([16, 48, 64, 100])
        frags = random_frags(rnd, P, rnd.randint(0, 30), 200)
        first = rnd.randint(0, 1000)
        got = _tiles(np.array(frags, dtype=np.int64).reshape(-1, 3), P, first)
        assert np.array_equal(got, tiles_ref(frags, first)), (trial, frags)
        assert np.array_equal(tiles_of(np.array(frags, dtype=np.int64).reshape(-1, 3), P), tiles_ref(frags)[:, :3])


def test_prune_matches_restatement():
    rnd = random.Random(1)
    for trial in range(400):
        P = rnd.choice([16, 64, 100])
        frags = random_frags(rnd, P, rnd.randint(1, 25), 60)
        n = sum(f[2] for f in frags)
        a = rnd.randint(0, n)
        c0 = rnd.randint(a, n)
        c = rnd.randint(0, n - c0)
        pt = PageTable(64, P)
        pt.frags = [np.array(frags, dtype=np.int64)]
        pt.free = []
        suffix, freed = pt.prune(0, a, c0, c)
        kept_ref, suffix_ref, freed_ref = prune_ref(frags, a, c0, c)
        # The kept list may keep fragment boundaries the restatement regroups; the tokens
        # it covers, and so every read of it, must agree.
        assert np.array_equal(token_slots(pt.frags[0].tolist()), token_slots(kept_ref)), trial
        assert np.array_equal(token_slots(suffix.tolist()), token_slots(suffix_ref)), trial
        assert freed == freed_ref, trial
        assert pt.free == freed_ref[::-1]
        assert pt.length(0) == a + c


def test_prune_merges_adjacent_pieces_and_keeps_fragments_otherwise():
    pt = PageTable(8, 64)
    pt.reserve(0, 200)  # pages 0..3: 64, 64, 64, 8
    before = pt.frags[0].copy()
    suffix, freed = pt.prune(0, 10, 10, 190)  # a == c0: nothing dropped
    assert np.array_equal(pt.frags[0], before) and freed == []
    assert np.array_equal(suffix, [[0, 10, 54], [1, 0, 64], [2, 0, 64], [3, 0, 8]])
    suffix, freed = pt.prune(0, 30, 140, 50)  # drop [30, 140): page 1 freed, page 0 and 2 cut
    assert np.array_equal(pt.frags[0], [[0, 0, 30], [2, 12, 50]])
    assert np.array_equal(suffix, [[2, 12, 50]])
    assert freed == [1, 3]
    suffix, freed = pt.prune(0, 0, 0, 0)  # keep nothing
    assert len(pt.frags[0]) == 0 and len(suffix) == 0 and freed == [0, 2]


def test_token_offsets_match_restatement():
    rnd = random.Random(2)
    for trial in range(100):
        P = rnd.choice([16, 64])
        pt = PageTable(300, P, batch=2)
        pt.frags = [np.array(random_frags(rnd, P, rnd.randint(0, 20), 300), dtype=np.int64).reshape(-1, 3)
                    for _ in range(2)]
        pitch = rnd.choice([None, 2000])
        off = pt.token_offsets(P * 256, 256, pitch)
        n = max([pt.length(b) for b in range(2)] + [1])
        assert off.shape == (2, max(n, pitch or 0)) and off.dtype == np.int32
        for b in range(2):
            sl = token_slots(pt.frags[b].tolist())
            want = np.full(off.shape[1], np.iinfo(np.int32).min, dtype=np.int64)
            want[:len(sl)] = sl[:, 0] * P * 256 + sl[:, 1] * 256
            assert np.array_equal(off[b], want), trial


def test_token_offsets_refuse_2gib():
    pt = PageTable(4, 64)
    pt.frags = [np.array([[3, 0, 64]], dtype=np.int64)]
    with pytest.raises(RuntimeError, match="2 GiB"):
        pt.token_offsets(1 << 30, 256)


def test_malformed_fragments_are_refused():
    lib = _lib.load()
    bad = np.array([[0, 5, 0]], dtype=np.int64)  # empty fragment
    assert lib.tc_page_tiles(bad.ctypes.data, 1, 64, 0, None, 0) == -_lib.TC_ERR_INVALID_ARGUMENT
    neg = np.array([[-1, 0, 4]], dtype=np.int64)
    assert lib.tc_page_tiles(neg.ctypes.data, 1, 64, 0, None, 0) == -_lib.TC_ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("frag", [[0, 60, 5], [0, 0, 65], [2, 64, 1], [1, -1, 3], [1, 3, 0]])
def test_fragments_past_their_page_are_refused(frag):
    """A fragment whose slots run past its page (first slot + count > page_tokens) would
    name rows of the next page or head: every page-table entry point refuses it."""
    lib = _lib.load()
    f = np.array([[3, 0, 16], frag], dtype=np.int64)
    INVALID = _lib.TC_ERR_INVALID_ARGUMENT
    assert lib.tc_page_tiles(f.ctypes.data, 2, 64, 0, None, 0) == -INVALID
    out = np.zeros(200, dtype=np.int32)
    assert lib.tc_page_token_offsets(f.ctypes.data, 2, 64, 64 * 256, 256, out.ctypes.data, 200) == -INVALID
    buf = np.zeros(64, dtype=np.int64)
    counts = np.zeros(3, dtype=np.int64)
    rc = lib.tc_page_prune(f.ctypes.data, 2, 64, 0, 0, 1, buf.ctypes.data, buf[20:].ctypes.data,
                           buf[40:].ctypes.data, counts.ctypes.data_as(_lib._I64P))
    assert rc == INVALID
    # The same list with the fragment inside its page is taken, and page_tokens < 1 is refused.
    ok = np.array([[3, 0, 16], [0, 48, 16]], dtype=np.int64)
    assert lib.tc_page_tiles(ok.ctypes.data, 2, 64, 0, None, 0) == 2
    assert lib.tc_page_tiles(ok.ctypes.data, 2, 0, 0, None, 0) == -INVALID
    assert lib.tc_page_tiles(ok.ctypes.data, 2, 63, 0, None, 0) == -INVALID
    pt = PageTable(4, 64)
    pt.frags = [np.array([[0, 0, 10]], dtype=np.int64)]
    with pytest.raises(ValueError):
        pt.prune(0, 5, 4, 1)
