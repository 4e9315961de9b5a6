"""The host planner of device-planned forwards (nanoslg_amd/csrc/host_plan.c, the
`_nslg_host` extension) against the numpy path it replaces (PagedCacheContext with
PagedKVCache.NATIVE_PLAN off), on the CPU with the stand-in kernels.

Two caches take the same random serving traffic, every forward of the numpy one
device-planned too (its token threshold lowered to 1): admissions on shared token prefixes (radix
matches, partial pages), ragged prefills with input offsets, decode rows, forwards
that copy shared pages (the native call declines those: the numpy path takes them),
deferred zeroing, releases, decode batches on shared prefixes (prefix groups). After
each begin_forward every plan array and prefix group, the pool's
refcounts, tokens_used and free stack, and the sequences' tables and device-row
marks must be equal; after attend the outputs and the pools' bytes.
The same traffic against the oracle is tests/test_host_random.py's
test_random_serving_traffic_device_planned."""
import random

import numpy as np
import pytest
import torch

import fake_kernels as FK
from nanoslg_amd import _lib
from nanoslg_amd import kv_cache as KC

L, HQ, HKV, D = 2, 4, 2, 8


def _cache(ps, pages, native):
    cfg = KC.KVCacheConfig(num_layers=L, num_kv_heads=HKV, num_qo_heads=HQ, head_dim=D, page_size=ps,
                           max_pages=pages, dtype=torch.float32, device=None, enable_prefix_caching=True,
                           backend="paged", share_partial_pages=True)
    c = KC.PagedKVCache(cfg, kernels=FK)
    c.NATIVE_PLAN = native
    return c


PLAN_FIELDS = ("slot", "pos_i32", "indptr", "indices", "lpl", "qo_indptr", "q_rows", "cow_src", "cow_dst", "zero_ids",
               "group_slot")


def _same_plan(p1, p2):
    for f in PLAN_FIELDS:
        a, b = getattr(p1, f, None), getattr(p2, f, None)
        if a is None or b is None:
            assert a is None and b is None, f
            continue
        if f == "zero_ids":
            # the native planner skips pages the forward writes in every slot (a decode
            # step at page size 1 fills the page it opens); the numpy decode path zeroes
            # them first: same pool bytes (checked after attend), a shorter list
            it = iter(b.tolist())
            assert all(z in it for z in a.tolist()), (a, b)
            continue
        assert torch.equal(a, b), (f, a, b)
    assert p1.total_pages == p2.total_pages and p1.total_q == p2.total_q
    g1, g2 = p1.groups, p2.groups
    assert (g1 is None) == (g2 is None)
    if g1 is not None:
        pp = lambda g: [int(x) for x in getattr(g, "prefix_pages_np", getattr(g, "prefix_pages", []))]  # noqa: E731
        assert g1.members == g2.members and pp(g1) == pp(g2)


def _same_state(a, b):
    assert np.array_equal(a.pool.ref_count, b.pool.ref_count)
    assert np.array_equal(a.pool.tokens_used, b.pool.tokens_used)
    assert a.pool._free == b.pool._free
    assert not a.pool._mark.any() and not b.pool._mark.any()
    assert a._pending_zero == b._pending_zero
    assert sorted(a.seqs) == sorted(b.seqs)
    for sid in a.seqs:
        s1, s2 = a.seqs[sid], b.seqs[sid]
        assert s1.n_pages == s2.n_pages and s1.num_tokens == s2.num_tokens
        assert np.array_equal(s1.bt[:s1.n_pages], s2.bt[:s2.n_pages])
        assert (s1.row, s1.row_cap, s1.synced) == (s2.row, s2.row_cap, s2.synced)
    assert torch.equal(a._tables.dev, b._tables.dev)


def _forward(a, b, ids, ntok, offs, g, stats):
    S = max(o + n for o, n in zip(offs, ntok))
    B = len(ids)
    q = torch.randn(B, S, HQ, D, generator=g)
    k = torch.randn(B, S, HKV, D, generator=g)
    v = torch.randn(B, S, HKV, D, generator=g)
    errs = []
    ctxs = []
    for c in (a, b):
        try:
            ctxs.append(c.begin_forward(ids, ntok, offs))
            errs.append(None)
        except RuntimeError as e:
            errs.append(str(e))
    assert errs[0] == errs[1]
    _same_state(a, b)
    if errs[0]:
        stats["oom"] += 1
        return False
    c1, c2 = ctxs
    _same_plan(c1._plan, c2._plan)
    assert c1.cow_pairs == c2.cow_pairs and c1._max_q == c2._max_q and c1._uniform_rows == c2._uniform_rows
    stats["cow" if c1.cow_pairs else "plain"] += 1
    for layer in range(L):
        o1 = c1.attend(layer, q, k, v, HQ, HKV)
        o2 = c2.attend(layer, q, k, v, HQ, HKV)
        assert torch.equal(o1, o2)
    a.end_forward(c1)
    b.end_forward(c2)
    assert torch.equal(a.pool.k, b.pool.k) and torch.equal(a.pool.v, b.pool.v)
    return True


@pytest.mark.parametrize("seed,ps,pages", [(1, 4, 64), (2, 1, 80), (3, 16, 16), (4, 3, 40), (5, 8, 24), (6, 2, 30)])
def test_native_plan_matches_the_numpy_plan(monkeypatch, seed, ps, pages):
    monkeypatch.setattr(KC.PagedCacheContext, "DEVICE_PLAN_TOKENS", 1)
    calls = {"n": 0}
    real = KC._host_planner

    def counted():
        f = real()

        def wrapped(*args):
            calls["n"] += 1
            return f(*args)
        return wrapped
    monkeypatch.setattr(KC, "_host_planner", counted)
    rnd = random.Random(seed)
    g = torch.Generator().manual_seed(seed)
    a, b = _cache(ps, pages, True), _cache(ps, pages, False)
    pending, running, tokens = {}, [], {}
    stats = {"plain": 0, "cow": 0, "oom": 0}
    for it in range(150):
        r = rnd.random()
        if r < 0.25 and len(pending) + len(running) < 6:
            sid = f"s{it}"
            toks = [rnd.randint(0, 2) for _ in range(rnd.randint(1, 4 * ps + 5))]
            if tokens and rnd.random() < 0.4:
                base = tokens[rnd.choice(sorted(tokens))]
                toks = base[:rnd.randint(1, len(base))] + toks[:rnd.randint(0, ps)]
            res = []
            for c in (a, b):
                try:
                    res.append(c.allocate_sequence(sid, token_ids=toks))
                except RuntimeError:
                    res.append(None)
            assert res[0] == res[1]
            _same_state(a, b)
            if res[0] is None:
                continue
            tokens[sid] = list(toks)
            if len(toks) > res[0]:
                pending[sid] = len(toks) - res[0]
            else:
                running.append(sid)
        elif r < 0.45 and pending:
            ids = sorted(pending)[: rnd.randint(1, len(pending))]
            ntok = [pending[s] for s in ids]
            # a chunk of the prompt, or all of it
            ntok = [n if rnd.random() < 0.6 else rnd.randint(1, n) for n in ntok]
            offs = [rnd.randint(0, 2) for _ in ids]
            if not _forward(a, b, ids, ntok, offs, g, stats):
                continue
            for s, n in zip(ids, ntok):
                pending[s] -= n
                if pending[s] == 0:
                    del pending[s]
                    running.append(s)
        elif r < 0.75 and running:
            ids = list(running)
            if rnd.random() < 0.3 and len(ids) > 1:
                ids = sorted(rnd.sample(ids, rnd.randint(1, len(ids) - 1)))
            ntok = [1] * len(ids)
            if pending and rnd.random() < 0.5:  # decode rows with prefill rows
                extra = sorted(pending)[:1]
                ids += extra
                ntok += [pending[extra[0]]]
            offs = [rnd.randint(0, 1) if n > 1 else 0 for n in ntok]
            if not _forward(a, b, ids, ntok, offs, g, stats):
                continue
            for s in ids:
                if s in pending:
                    del pending[s]
                    running.append(s)
                else:
                    t = rnd.randint(0, 2)
                    tokens[s].append(t)
                    a.append_token_ids(s, [t])
                    b.append_token_ids(s, [t])
        elif r < 0.85 and running:
            # another sequence on a running one's pages, its last partial page included:
            # the next write of either copies it (copy-on-write: the numpy path)
            src = rnd.choice(running)
            n = a.seqs[src].num_tokens
            if n == 0 or n % ps == 0:
                continue
            sid = f"c{it}"
            for c in (a, b):
                c.allocate_sequence(sid)
                pages_ = c.seqs[src].block_table[: (n + ps - 1) // ps]
                for p in pages_:
                    c.pool.add_ref(p)
                c.seqs[sid].extend(pages_)
                c.seqs[sid].num_tokens = n
            tokens[sid] = list(tokens[src][:n])
            running.append(sid)
        elif running or pending:
            sid = rnd.choice(running + sorted(pending))
            a.release_sequence(sid)
            b.release_sequence(sid)
            pending.pop(sid, None)
            if sid in running:
                running.remove(sid)
        _same_state(a, b)
    assert stats["plain"] >= 10 and calls["n"] >= 10, (stats, calls)


def test_native_plan_declines_a_shared_write_and_changes_nothing():
    """A forward that writes a page with refcount > 1 gets None from the planner and
    no state changes (the copy-on-write path then runs in Python)."""
    c = _cache(4, 32, True)
    c.allocate_sequence("a")
    ctx = c.begin_forward(["a"], [6])  # pages 0..1, the second partial
    c.end_forward(ctx)
    st = c.seqs["a"]
    c.pool.add_ref(int(st.bt[1]))
    c.extend_sequence("a", 3)
    used = c.pool.tokens_used.copy()
    rows = (st.row, st.row_cap, st.synced)
    placed = []
    out = np.full(256, -7, np.int32)
    res = _lib.host().plan_forward([st], [3], [0], 4, c.pool.ref_count, c.pool.tokens_used, c.pool._mark, None, out,
                                   placed.append)
    assert res is None and not placed
    assert np.array_equal(c.pool.tokens_used, used) and (out == -7).all() and (st.row, st.row_cap, st.synced) == rows


def test_native_plan_asks_for_a_larger_buffer_and_changes_nothing():
    c = _cache(4, 64, True)
    c.allocate_sequence("a")
    c.extend_sequence("a", 40)
    st = c.seqs["a"]
    used = c.pool.tokens_used.copy()
    out = np.zeros(8, np.int32)
    res = _lib.host().plan_forward([st], [40], None, 4, c.pool.ref_count, c.pool.tokens_used, c.pool._mark,
                                   list(c._pending_zero), out, c._tables.place)
    assert isinstance(res, int) and res < -8
    assert np.array_equal(c.pool.tokens_used, used) and not out.any() and st.row < 0
    big = np.zeros(-res, np.int32)
    total, total_pages, npatch, nz, shared_first = _lib.host().plan_forward(
        [st], [40], None, 4, c.pool.ref_count, c.pool.tokens_used, c.pool._mark, list(c._pending_zero), big,
        c._tables.place)
    # 40 tokens on 10 fresh pages, all written whole: nothing left to zero; the sequence
    # got its device row, all 10 entries due
    assert (total_pages, npatch, nz, shared_first) == (10, 10, 0, False) and total == -res - len(c._pending_zero)
    assert st.row >= 0
    assert big[:2].tolist() == [0, 10] and big[2] == 4  # kv_indptr, last page length
    assert c.pool.tokens_used[st.bt[:10]].tolist() == [4] * 10


def test_native_plan_rejects_bad_arguments():
    plan = _lib.host().plan_forward
    rc, tu, mk = np.zeros(8, np.int64), np.zeros(8, np.int64), np.zeros(8, bool)
    f = lambda s: None  # noqa: E731
    with pytest.raises(TypeError):
        plan((), [], None, 4, rc, tu, mk, None, np.zeros(8, np.int32), f)
    with pytest.raises(ValueError):
        plan([], [1], None, 4, rc, tu, mk, None, np.zeros(8, np.int32), f)
    with pytest.raises(ValueError):
        plan([], [], None, 0, rc, tu, mk, None, np.zeros(8, np.int32), f)
    with pytest.raises(TypeError):
        plan([], [], None, 4, rc, tu, mk, None, np.zeros(8, np.int64), f)  # out must be int32
    with pytest.raises(ValueError):
        plan([], [], None, 4, rc, np.zeros(4, np.int64), mk, None, np.zeros(8, np.int32), f)
    with pytest.raises(TypeError):
        plan([], [], None, 4, rc, tu, mk, None, np.zeros(8, np.int32), None)  # place must be callable
    with pytest.raises(TypeError):
        plan([], [], None, 4, rc, tu, mk, None, np.zeros(8, np.int32))  # 9 arguments


def test_native_plan_rejects_out_of_range_sequences():
    """A state whose token count is negative, or whose tokens would not fit the plan's
    int32 positions, is refused before anything is read or written."""
    import types
    plan = _lib.host().plan_forward
    rc, tu, mk = np.zeros(8, np.int64), np.zeros(8, np.int64), np.zeros(8, bool)
    out = np.zeros(256, np.int32)
    placed = []
    for num_tokens, n in ((-1, 4), (0, 1 << 31), ((1 << 31) - 2, 4)):
        st = types.SimpleNamespace(num_tokens=num_tokens, n_pages=1, bt=np.array([1, 0], np.int32), row=-1,
                                   synced=0)
        with pytest.raises(ValueError, match="out of range"):
            plan([st], [n], None, 4, rc, tu, mk, None, out, placed.append)
    assert not placed and not tu.any() and not out.any()


def test_native_plan_places_only_rows_that_are_missing_or_short():
    """The planner calls `place` for a state without a device row or with one shorter
    than its table, and for no other: a steady forward makes no callback."""
    c = _cache(4, 64, True)
    for s in ("a", "b"):
        c.allocate_sequence(s)
    c.extend_sequence("a", 8)
    c.extend_sequence("b", 3)
    sa, sb = c.seqs["a"], c.seqs["b"]
    plan = _lib.host().plan_forward
    calls = []

    def place(st):
        calls.append(st.seq_id)
        c._tables.place(st)

    def run(states, ntoks):
        out = np.zeros(4096, np.int32)
        res = plan(states, ntoks, None, 4, c.pool.ref_count, c.pool.tokens_used, c.pool._mark, None, out, place)
        assert isinstance(res, tuple)
        for st in states:  # what the cache does after the plan's upload
            st.synced = st.n_pages
        return res

    run([sa, sb], [8, 3])  # no rows yet: both placed
    assert calls == ["a", "b"] and sa.row >= 0 and sb.row >= 0
    for st, n in ((sa, 8), (sb, 3)):
        st.num_tokens += n
    del calls[:]
    run([sa, sb], [1, 1])  # the rows hold the tables: no callback
    assert calls == []
    cap = sb.row_cap
    c.extend_sequence("b", 4 * cap)  # b's table outgrows its row
    run([sa, sb], [0, 4 * cap])
    assert calls == ["b"] and sb.row_cap >= sb.n_pages
