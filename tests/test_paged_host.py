"""Paged cache bookkeeping on the CPU: PageTable against a brute-force model
that tracks the (page, slot) of every token, through random appends and
prunes of several sequences."""
import random

import numpy as np
import pytest

from threadcut_amd.paged import TILE, PageTable, tiles_of


def check_table(t, model):
    used = set()
    for b in range(t.batch):
        slots = [tuple(x) for x in t.token_slots(b).tolist()]
        assert slots == model[b]
        assert t.length(b) == len(model[b])
        for page, slot in slots:
            assert 0 <= page < t.num_pages and 0 <= slot < t.page_tokens
            assert (page, slot) not in used
            used.add((page, slot))
    pages_used = {p for p, _ in used}
    # A page is free exactly when no kept token uses it.
    assert sorted(t.free) == sorted(set(range(t.num_pages)) - pages_used)
    assert len(t.free) == len(set(t.free))
    tab, cnt = t.tile_table()
    for b in range(t.batch):
        ts = tiles_of(t.frags[b], t.page_tokens).tolist()
        assert cnt[b] == len(ts)
        rows = []
        for (page, slot, n), e in zip(ts, tab[b].tolist()):
            assert tuple(e) == (page, slot, n, len(rows))  # the 4th word: the tile's first logical position
            assert 1 <= n <= TILE and slot + n <= t.page_tokens
            assert slot // TILE == (slot + n - 1) // TILE  # a tile never crosses a 16-slot boundary
            rows += [(page, slot + i) for i in range(n)]
        assert rows == model[b]
    # Byte offsets of every token's row in a head slab (page stride 1000 B, slot stride 10 B here).
    off = t.token_offsets(1000, 10, pitch=5)
    assert off.dtype == np.int32 and off.shape[1] >= max([5] + [len(m) for m in model])
    for b in range(t.batch):
        want = [p * 1000 + s_ * 10 for p, s_ in model[b]]
        assert off[b, :len(want)].tolist() == want
        assert (off[b, len(want):] == np.iinfo(np.int32).min).all()


@pytest.mark.parametrize("page_tokens", [16, 64, 40])
@pytest.mark.parametrize("seed", range(6))
def test_page_table_matches_brute_force(page_tokens, seed):
    rnd = random.Random(seed)
    batch = 3
    t = PageTable(num_pages=400, page_tokens=page_tokens, batch=batch)
    model = [[] for _ in range(batch)]
    for _ in range(60):
        b = rnd.randrange(batch)
        if rnd.random() < 0.6 or not model[b]:
            n = rnd.choice([0, 1, 1, 2, 7, 16, 33, rnd.randint(1, 300)])
            if len(t.free) * page_tokens < n + page_tokens:
                continue
            got = t.reserve(b, n)
            assert len(got) == n
            model[b] += [tuple(x) for x in got.tolist()]
        else:
            length = len(model[b])
            a = rnd.randint(0, length)
            c0 = rnd.randint(a, length)
            c = rnd.randint(0, length - c0)
            suffix, freed = t.prune(b, a, c0, c)
            want_suffix = model[b][c0:c0 + c]
            assert [(p, s + i) for p, s, n in suffix.tolist() for i in range(n)] == want_suffix
            model[b] = model[b][:a] + want_suffix
            assert all(p not in {q for q, _ in model[b]} for p in freed)
        check_table(t, model)
    for b in range(batch):
        t.release(b)
        model[b] = []
        check_table(t, model)
    assert len(t.free) == t.num_pages


def test_prune_frees_whole_pages_of_the_span():
    t = PageTable(num_pages=20, page_tokens=16, batch=1)
    t.reserve(0, 160)  # pages 0..9
    suffix, freed = t.prune(0, 20, 100, 60)  # keep [0,20) and [100,160)
    assert freed == [2, 3, 4, 5]  # tokens 32..95 only
    assert suffix.tolist() == [[6, 4, 12], [7, 0, 16], [8, 0, 16], [9, 0, 16]]
    assert t.frags[0].tolist() == [[0, 0, 16], [1, 0, 4]] + suffix.tolist()
    # The last page is full, so the next token takes a page the prune freed.
    assert t.reserve(0, 1).tolist() == [[2, 0]]
    t2 = PageTable(num_pages=4, page_tokens=16)
    t2.reserve(0, 20)
    t2.prune(0, 3, 10, 10)  # one page keeps both sides of the hole
    assert t2.frags[0].tolist() == [[0, 0, 3], [0, 10, 6], [1, 0, 4]]
    assert t2.reserve(0, 2).tolist() == [[1, 4], [1, 5]]


def test_reserve_and_prune_reject_bad_requests():
    t = PageTable(num_pages=2, page_tokens=16)
    with pytest.raises(RuntimeError, match="pages needed"):
        t.reserve(0, 33)
    assert t.length(0) == 0 and len(t.free) == 2
    t.reserve(0, 10)
    with pytest.raises(ValueError):
        t.prune(0, 5, 4, 1)
    with pytest.raises(ValueError):
        t.prune(0, 2, 5, 6)
    tab, cnt = PageTable(3, 16, batch=2).tile_table()
    assert tab.shape == (2, 1, 4) and not tab.any() and list(cnt) == [0, 0]


def test_paged_cache_rejects_host_pools():
    import torch

    from threadcut_amd.paged import PagedKV

    with pytest.raises(RuntimeError, match="GPU"):
        PagedKV(2, 8, 10, 16, device="cpu")
    with pytest.raises(TypeError):
        PagedKV(2, 8, 10, 16, dtype=torch.float32, device="cuda")
