"""Host layer (nanoslg_amd.kv_cache) against the CPU oracle on identical call
sequences. The HIP kernels are replaced by tests/fake_kernels.py so the
bookkeeping (allocation, block tables, copy-on-write order, radix sharing,
eviction, plans, positions) is checked on the CPU; the GPU tests run the same
host layer on the real kernels."""
import math
import random
import types

import numpy as np
import pytest
import torch

import fake_kernels as FK
from nanoslg_amd import kv_cache as KC
from oracle import kv_oracle as O

L, HQ, HKV, D = 2, 4, 2, 8


def make(ps=4, pages=64, prefix=True, dtype=torch.float32, partial=True):
    cfg = KC.KVCacheConfig(num_layers=L, num_kv_heads=HKV, num_qo_heads=HQ, head_dim=D, page_size=ps,
                           max_pages=pages, dtype=dtype, device=None, enable_prefix_caching=prefix,
                           backend="paged", share_partial_pages=partial)
    mgr = KC.PagedKVCache(cfg, kernels=FK)
    ref = O.PagedRef(L, pages, ps, HKV, D, dtype, enable_prefix_caching=prefix, share_partial_pages=partial)
    return mgr, ref


def logical(mgr, sid, layer):
    st = mgr.seqs[sid]
    ps = mgr.cfg.page_size
    n = st.num_tokens
    bt = st.block_table
    k = torch.stack([mgr.pool.k[layer, bt[t // ps], t % ps] for t in range(n)]) if n else None
    v = torch.stack([mgr.pool.v[layer, bt[t // ps], t % ps] for t in range(n)]) if n else None
    return k, v


def forward_both(mgr, ref, ids, ntok, offs, g):
    S = max(o + n for o, n in zip(offs, ntok))
    B = len(ids)
    q = torch.randn(B, S, HQ, D, generator=g)
    k = torch.randn(B, S, HKV, D, generator=g)
    v = torch.randn(B, S, HKV, D, generator=g)
    c1 = mgr.begin_forward(ids, ntok, offs)
    c2 = ref.begin_forward(ids, ntok, offs)
    assert c1.start_positions == c2.start_positions and c1.seq_lens == c2.seq_lens
    assert torch.equal(c1.get_position_ids(S), c2.get_position_ids(S))
    assert len(c1.cow_pairs) == len(c2.cow_events)
    for layer in range(L):
        o1 = c1.attend(layer, q, k, v, HQ, HKV)
        o2 = c2.attend(layer, q, k, v, HQ, HKV)
        assert o1.shape == (B, S, HQ * D)
        for b in range(B):
            rows = slice(offs[b], offs[b] + ntok[b])
            torch.testing.assert_close(o1[b, rows].float(), o2[b, rows], atol=1e-5, rtol=1e-5)
            # rows without a new token are zero
            pad = torch.ones(S, dtype=torch.bool)
            pad[rows] = False
            assert not o1[b, pad].any()
    mgr.end_forward(c1)
    ref.end_forward(c2)
    return c1, c2


def check_state(mgr, ref, ids):
    assert mgr.pool.num_free == ref.pool.num_free
    for sid in ids:
        assert mgr.seqs[sid].num_tokens == ref.seqs[sid].num_tokens
        for layer in range(L):
            k1, v1 = logical(mgr, sid, layer)
            k2, v2 = ref.logical_kv(sid, layer)
            if k1 is None:
                assert k2.shape[0] == 0
                continue
            assert torch.equal(k1, k2) and torch.equal(v1, v2)


def test_prefill_then_decode_matches_oracle():
    g = torch.Generator().manual_seed(0)
    mgr, ref = make()
    ids = ["a", "b", "c"]
    lens = [5, 9, 3]
    for s, n in zip(ids, lens):
        assert mgr.allocate_sequence(s, num_tokens=n) == ref.allocate_sequence(s, num_tokens=n) == 0
    forward_both(mgr, ref, ids, lens, [max(lens) - n for n in lens], g)  # left-padded prefill
    check_state(mgr, ref, ids)
    for _ in range(9):
        forward_both(mgr, ref, ids, [1, 1, 1], [0, 0, 0], g)
    check_state(mgr, ref, ids)
    # chunked prefill step of uneven sizes, including a sequence with no new tokens
    forward_both(mgr, ref, ids, [3, 0, 6], [3, 6, 0], g)
    check_state(mgr, ref, ids)


def test_positions_shapes():
    mgr, _ = make()
    mgr.allocate_sequence("a", num_tokens=3)
    mgr.allocate_sequence("b", num_tokens=2)
    ctx = mgr.begin_forward(["a", "b"], [3, 2], [0, 1])
    assert ctx.get_position_ids(3).tolist() == [[0, 1, 2], [0, 0, 1]]
    assert ctx.get_position_ids(2).tolist() == [[0, 1], [0, 0]]
    assert ctx.get_position_ids(5).tolist() == [[0, 1, 2, 0, 0], [0, 0, 1, 0, 0]]
    assert ctx.get_position_ids(3).dtype == torch.long
    assert ctx.get_start_pos(1) == 0 and ctx.get_position(3).shape == (2, 3)


def test_csr_plan_closed_form():
    mgr, _ = make(ps=4)
    mgr.allocate_sequence("a", num_tokens=9)
    mgr.allocate_sequence("b", num_tokens=4)
    mgr.seqs["a"].num_tokens = 9
    mgr.seqs["b"].num_tokens = 4
    ctx = mgr.begin_forward(["a", "b"], [1, 1])
    plan = ctx.plan
    bt_a, bt_b = mgr.seqs["a"].block_table, mgr.seqs["b"].block_table
    assert plan.indptr.tolist() == [0, 3, 5]
    assert plan.indices.tolist() == bt_a[:3] + bt_b[:2]
    assert plan.lpl.tolist() == [2, 1]
    assert plan.slot.tolist() == [bt_a[2] * 4 + 1, bt_b[1] * 4 + 0]
    assert plan.total_pages == 5


def _share_page(mgr_or_ref, ids, page, tokens):
    """Make `ids` share one page holding `tokens` tokens (refcount = len(ids))."""
    for s in ids:
        st = mgr_or_ref.seqs[s]
        if isinstance(st, KC._PagedSeqState):
            st.set_page(0, page)
            st.n_pages = 1
        else:
            st.block_table = [page]
        st.num_tokens = tokens


def test_copy_on_write_order_rule():
    """Refcount R held by R sharers: the first R-1 writers copy, the last writes in place."""
    g = torch.Generator().manual_seed(1)
    for mgr_ref in [make(prefix=False)]:
        mgr, ref = mgr_ref
        ids = ["x", "y", "z"]
        for s in ids:
            mgr.allocate_sequence(s, num_tokens=1)
            ref.allocate_sequence(s, num_tokens=1)
        # both: seq x's page becomes the shared one, the others' pages are released
        for impl in (mgr, ref):
            shared = impl.seqs["x"].block_table[0]
            for s in ["y", "z"]:
                impl.pool.release(impl.seqs[s].block_table[0])
                impl.pool.add_ref(shared)
            impl.pool.k[:, shared] = 3.0
            impl.pool.v[:, shared] = -1.0
            _share_page(impl, ids, shared, 2)
        assert mgr.pool.ref_count[mgr.seqs["x"].block_table[0]] == 3
        c1, c2 = forward_both(mgr, ref, ids, [1, 1, 1], [0, 0, 0], g)
        assert len(c1.cow_pairs) == 2
        src = c1.cow_pairs[0][0]
        assert [p[0] for p in c1.cow_pairs] == [src, src]
        assert mgr.seqs["z"].block_table[0] == src        # last sharer writes in place
        assert mgr.pool.ref_count[src] == 1
        check_state(mgr, ref, ids)
        # copied pages carry the source's tokens_used and the source's bytes beyond slot 2
        for s in ["x", "y"]:
            p = mgr.seqs[s].block_table[0]
            assert mgr.pool.tokens_used[p] == 3
            assert torch.equal(mgr.pool.k[:, p, 3], mgr.pool.k[:, src, 3])


def test_cow_oom_raises():
    mgr, _ = make(prefix=False, pages=4)
    mgr.allocate_sequence("x", num_tokens=1)
    mgr.allocate_sequence("y", num_tokens=1)
    mgr.allocate_sequence("z", num_tokens=1)
    shared = mgr.seqs["x"].block_table[0]
    for s in ["y", "z"]:
        mgr.pool.release(mgr.seqs[s].block_table[0])
        mgr.pool.add_ref(shared)
    _share_page(mgr, ["x", "y", "z"], shared, 2)
    mgr.allocate_sequence("w", num_tokens=8)  # takes the two free pages
    with pytest.raises(RuntimeError, match="KV OOM during CoW"):
        mgr.begin_forward(["x"], [1])


def test_cow_oom_keeps_the_copies_already_made():
    """Three sequences share a partial page; the pool holds one more page. A decode
    forward of all three copies the page for the first writer, then runs out at the
    second: RuntimeError, as in the reference, whose first copy already happened
    (kv_cache.py:429-436, 586-591). The first sequence reads the same K/V as before,
    through its new page, on both sides."""
    g = torch.Generator().manual_seed(11)
    mgr, ref = make(ps=4, pages=6, prefix=False)
    for impl in (mgr, ref):
        impl.allocate_sequence("a")
    forward_both(mgr, ref, ["a"], [6], [0], g)          # pages: 4 tokens + 2 in a partial page
    for impl in (mgr, ref):
        st = impl.seqs["a"]
        pages = list(st.block_table)
        for sid in ("b", "c"):
            impl.allocate_sequence(sid)
            for p in pages:
                impl.pool.add_ref(p)
            nst = impl.seqs[sid]
            if hasattr(nst, "bt"):
                nst.extend(pages)
            else:
                nst.block_table = list(pages)
            nst.num_tokens = 6
        impl.allocate_sequence("filler", num_tokens=8)  # two of the three free pages
    assert mgr.pool.num_free == ref.pool.num_free == 1
    before = logical(mgr, "a", 0)
    with pytest.raises(RuntimeError, match="KV OOM during CoW"):
        mgr.begin_forward(["a", "b", "c"], [1, 1, 1])
    with pytest.raises(RuntimeError, match="KV OOM during CoW"):
        ref.begin_forward(["a", "b", "c"], [1, 1, 1])
    assert mgr.seqs["a"].block_table[-1] != mgr.seqs["b"].block_table[-1]  # a moved to its copy
    after = logical(mgr, "a", 0)
    assert torch.equal(before[0], after[0]) and torch.equal(before[1], after[1])
    check_state(mgr, ref, ["a", "b", "c"])


def test_kv_oom_message_and_eviction():
    mgr, ref = make(pages=6, prefix=True)
    with pytest.raises(RuntimeError, match=r"KV OOM: need 6, free 5"):
        mgr.allocate_sequence("big", num_tokens=24)
    with pytest.raises(RuntimeError, match=r"KV OOM: need 6, free 5"):
        ref.allocate_sequence("big", num_tokens=24)
    # fill the tree with cached pages, then allocation must evict them
    g = torch.Generator().manual_seed(2)
    toks = list(range(100, 116))
    for impl in (mgr, ref):
        impl.allocate_sequence("a", token_ids=toks)
    forward_both(mgr, ref, ["a"], [16], [0], g)
    mgr.release_sequence("a")
    ref.release_sequence("a")
    assert mgr.tree.cached_pages == ref.tree.cached_pages == 4
    assert mgr.pool.num_free == ref.pool.num_free == 1
    assert mgr.allocate_sequence("b", num_tokens=12) == 0
    ref.allocate_sequence("b", num_tokens=12)
    assert mgr.pool.num_free == ref.pool.num_free
    assert mgr.tree.cached_pages == ref.tree.cached_pages


@pytest.mark.parametrize("partial", [False, True])
def test_radix_prefix_sharing_matches_oracle(partial):
    """Full pages shared through the tree (kv_cache.py:459-486); with partial-page
    sharing the released sequence's last page (one token) is cached too."""
    g = torch.Generator().manual_seed(3)
    mgr, ref = make(ps=4, pages=64, prefix=True, partial=partial)
    prompt = [7, 1, 3, 3, 9, 9, 2, 5, 4, 4, 6, 8, 1, 2]  # 3 full pages + 2 tokens
    for impl in (mgr, ref):
        assert impl.allocate_sequence("p", token_ids=prompt) == 0
    forward_both(mgr, ref, ["p"], [len(prompt)], [0], g)
    for _ in range(3):
        forward_both(mgr, ref, ["p"], [1], [0], g)
        for impl in (mgr, ref):
            impl.append_token_ids("p", [11])
    mgr.release_sequence("p")
    ref.release_sequence("p")
    assert mgr.tree.cached_pages == ref.tree.cached_pages == 4 + int(partial)  # 17 tokens: 4 full pages + 1
    # a new request sharing the first 2 pages, then diverging
    q = prompt[:8] + [0, 0, 0, 0, 0]
    p1 = mgr.allocate_sequence("q", token_ids=q)
    p2 = ref.allocate_sequence("q", token_ids=q)
    assert p1 == p2 == 8
    # the cache's first two logical pages hold the same K/V as the prompt had
    check_state(mgr, ref, ["q"])
    forward_both(mgr, ref, ["q"], [len(q) - 8], [0], g)
    check_state(mgr, ref, ["q"])
    forward_both(mgr, ref, ["q"], [1], [0], g)
    check_state(mgr, ref, ["q"])
    mgr.release_sequence("q")
    ref.release_sequence("q")
    assert mgr.pool.num_free == ref.pool.num_free


def test_radix_random_workload_matches_oracle():
    """Random admissions over a small vocabulary: prefix hits, inserts and evictions."""
    rnd = random.Random(5)
    g = torch.Generator().manual_seed(5)
    mgr, ref = make(ps=2, pages=40, prefix=True)
    live = {}
    for it in range(60):
        if live and (rnd.random() < 0.4 or len(live) >= 3):
            sid = rnd.choice(sorted(live))
            mgr.release_sequence(sid)
            ref.release_sequence(sid)
            del live[sid]
        else:
            sid = f"r{it}"
            toks = [rnd.randint(0, 2) for _ in range(rnd.randint(2, 9))]
            try:
                p1 = mgr.allocate_sequence(sid, token_ids=toks)
            except RuntimeError:
                with pytest.raises(RuntimeError):
                    ref.allocate_sequence(sid, token_ids=toks)
                continue
            p2 = ref.allocate_sequence(sid, token_ids=toks)
            assert p1 == p2
            n = len(toks) - p1
            if n > 0:
                forward_both(mgr, ref, [sid], [n], [0], g)
            live[sid] = toks
        assert mgr.pool.num_free == ref.pool.num_free
        assert mgr.tree.cached_pages == ref.tree.cached_pages
        check_state(mgr, ref, sorted(live))


def test_decode_batch_with_new_pages_zeroed():
    g = torch.Generator().manual_seed(6)
    mgr, ref = make(ps=4)
    ids = ["a", "b"]
    for impl in (mgr, ref):
        impl.allocate_sequence("a", num_tokens=4)
        impl.allocate_sequence("b", num_tokens=3)
    forward_both(mgr, ref, ids, [4, 3], [0, 1], g)
    FK.CALLS.clear()
    forward_both(mgr, ref, ids, [1, 1], [0, 0], g)  # "a" crosses into a new page
    assert [c for c in FK.CALLS if c[0] == "zero_pages"] == [("zero_pages", 1)]
    p = mgr.seqs["a"].block_table[1]
    assert not mgr.pool.k[:, p, 1:].any()
    check_state(mgr, ref, ids)


def test_contiguous_backend_matches_oracle():
    g = torch.Generator().manual_seed(7)
    cfg = KC.KVCacheConfig(num_layers=L, num_kv_heads=HKV, num_qo_heads=HQ, head_dim=D, max_batch_size=3,
                           max_seq_len=32, dtype=torch.float32, device=None, backend="contiguous")
    mgr = KC.ContiguousKVCache(cfg, kernels=FK)
    ref = O.ContiguousRef(L, 3, 32, HKV, D)
    ids = ["a", "b", "c"]
    for s in ids:
        mgr.allocate_sequence(s)
        ref.allocate_sequence(s)
    steps = [([5, 9, 3], [4, 0, 6])] + [([1, 1, 1], [0, 0, 0])] * 5
    for ntok, offs in steps:
        S = max(o + n for o, n in zip(offs, ntok))
        q = torch.randn(3, S, HQ, D, generator=g)
        k = torch.randn(3, S, HKV, D, generator=g)
        v = torch.randn(3, S, HKV, D, generator=g)
        c1 = mgr.begin_forward(ids, ntok, offs)
        c2 = ref.begin_forward(ids, ntok, offs)
        assert torch.equal(c1.get_position_ids(S), c2.get_position_ids(S))
        for layer in range(L):
            o1 = c1.attend(layer, q, k, v, HQ, HKV)
            o2 = c2.attend(layer, q, k, v, HQ, HKV)
            for b in range(3):
                rows = slice(offs[b], offs[b] + ntok[b])
                torch.testing.assert_close(o1[b, rows], o2[b, rows], atol=1e-5, rtol=1e-5)
        mgr.end_forward(c1)
        ref.end_forward(c2)
    assert torch.equal(mgr.k, ref.k) and torch.equal(mgr.v, ref.v)
    assert mgr.stats["slots"] == "3/3"
    with pytest.raises(AssertionError):
        mgr.allocate_sequence("d")
    mgr.reset()
    assert mgr.stats["active_seqs"] == 0 and mgr.stats["slots"] == "0/3"


def test_config_and_factory():
    hf = types.SimpleNamespace(num_hidden_layers=32, num_key_value_heads=8, num_attention_heads=32,
                               hidden_size=4096)
    par = types.SimpleNamespace(tp_size=2, pp_size=1, pp_layer_splits=None)
    cfg = KC.KVCacheConfig.from_hf_config(hf, par, device=None, dtype=torch.float16)
    assert (cfg.num_layers, cfg.num_kv_heads, cfg.num_qo_heads, cfg.head_dim) == (32, 4, 16, 128)
    assert cfg.backend == "paged" and cfg.max_pages == 256  # no device -> the reference's default
    assert KC.KVCacheConfig(1, 8, 32, 128, backend="flashinfer", device=None).backend == "paged"
    with pytest.raises(ValueError):
        KC.KVCacheConfig(1, 8, 32, 128, backend="bogus")
    hf1 = types.SimpleNamespace(num_hidden_layers=2, num_key_value_heads=2, num_attention_heads=4,
                                hidden_size=32)
    m = types.SimpleNamespace(kv_backend="contiguous", max_seq_len=64)
    mgr = KC.create_cache_manager(hf1, None, "cpu", torch.float16, m, max_batch_size=2)
    assert isinstance(mgr, KC.ContiguousKVCache) and mgr.stats["max_seq"] == 64
    assert mgr.k.shape == (2, 2, 64, 2, 8)
    m = types.SimpleNamespace(page_size=8)  # kv_backend defaults to auto -> paged
    mgr = KC.create_cache_manager(hf1, None, "cpu", torch.float16, m)
    assert isinstance(mgr, KC.PagedKVCache) and mgr.pool.k.shape == (2, 256, 8, 2, 8)


def test_release_many_equals_one_release_per_page():
    """PagePool.release_many (used when a sequence is released) leaves the same
    refcounts, tokens_used, free flags and free-list order as release() page by page,
    with shared pages, page 0 and repeated ids in the list."""
    rng = np.random.default_rng(4)
    for trial in range(20):
        pools = [make(ps=4, pages=64, prefix=False)[0].pool for _ in range(2)]
        pages = pools[0].alloc(40, zero=False)
        assert pools[1].alloc(40, zero=False) == pages
        for pool in pools:
            for p in pages[::3]:
                pool.add_ref(p)
            pool.tokens_used[pages] = np.arange(40) % 4 + 1
        sel = rng.choice(pages, size=int(rng.integers(1, 40)), replace=bool(trial % 2)).tolist() + [0]
        rng.shuffle(sel)
        for p in sel:
            pools[0].release(p)
        pools[1].release_many(sel)
        a, b = pools
        assert np.array_equal(a.ref_count, b.ref_count) and np.array_equal(a.tokens_used, b.tokens_used)
        assert np.array_equal(a._is_free, b._is_free) and a._free == b._free


def test_unsupported_head_dim_is_rejected_at_construction():
    """A GPU cache whose dtype and head_dim some kernel it uses does not support (64,
    128 and 256 for every pool dtype) is refused when it is built, not at its first
    prefill."""
    from nanoslg_amd import kernels as K
    for dt, hd, ok in ((torch.float16, 96, False), (torch.bfloat16, 96, False), (torch.float32, 32, False),
                       (torch.float16, 128, True), (torch.float16, 256, True), (torch.bfloat16, 256, True),
                       (torch.float32, 256, True), (torch.bfloat16, 64, True)):
        cfg = KC.KVCacheConfig(1, 2, 4, hd, page_size=16, max_pages=8, dtype=dt, device=None)
        cfg.device = torch.device("cuda", 0)  # the check only; nothing is allocated here
        if ok:
            KC._check_head_dim(cfg, K)
        else:
            with pytest.raises(ValueError, match="head_dim"):
                KC._check_head_dim(cfg, K)


def test_stats_and_reset():
    mgr, _ = make(ps=4, pages=16, prefix=True)
    mgr.allocate_sequence("a", token_ids=list(range(9)))
    st = mgr.stats
    assert st["backend"] == "paged" and st["active_seqs"] == 1 and st["pages_used"] == 3
    mgr.seqs["a"].num_tokens = 9
    mgr.reset()
    # the tree keeps the 2 full pages and the partial third one (1 token)
    assert mgr.stats["active_seqs"] == 0 and mgr.stats["radix"] == 3 and mgr.pool.num_free == 12


@pytest.mark.parametrize("scalar_batch", [16, 0])
def test_device_decode_plan_matches_host_plan(scalar_batch, monkeypatch):
    """Steady decode steps build their plan from the previous one (decode_plan_step);
    each such plan equals, entry for entry, the plan the host builds for the same
    step, and pages, refcounts and tokens_used stay identical. Batch changes, prefill
    and shared pages fall back to the host plan. Both host checks of a step run: the
    per-sequence one of small batches (begin_forward's one-pass steady step) and the
    vectorised one."""
    monkeypatch.setattr(KC.PagedKVCache, "SCALAR_PLAN_BATCH", scalar_batch)
    monkeypatch.setattr(KC.PagedKVCache, "ONE_PASS_BATCH", scalar_batch)
    g = torch.Generator().manual_seed(11)
    fast, _ = make(ps=4, pages=96, prefix=False)
    slow, _ = make(ps=4, pages=96, prefix=False)
    slow._advance_decode_plan = lambda *a: None
    slow._begin_steady_decode = lambda *a: None
    ids = ["a", "b", "c", "d"]
    for m in (fast, slow):
        for s, n in zip(ids, [5, 8, 1, 3]):
            m.allocate_sequence(s, num_tokens=n)

    def step(ntok, sids, expect_fast=None):
        S = max(ntok)
        B = len(sids)
        q = torch.randn(B, S, HQ, D, generator=g)
        k = torch.randn(B, S, HKV, D, generator=g)
        v = torch.randn(B, S, HKV, D, generator=g)
        FK.CALLS.clear()
        c1 = fast.begin_forward(sids, ntok)
        used_fast = any(name == "decode_plan_step" for name, _ in FK.CALLS)
        c2 = slow.begin_forward(sids, ntok)
        if expect_fast is not None:
            assert used_fast == expect_fast
        p1, p2 = c1.plan, c2.plan
        for name in ("indptr", "indices", "lpl", "slot", "pos_i32", "zero_ids"):
            a, b = getattr(p1, name), getattr(p2, name)
            assert torch.equal(a.to(torch.int64), b.to(torch.int64)), name
        assert p1.total_pages == p2.total_pages
        o1 = c1.attend(0, q, k, v, HQ, HKV)
        o2 = c2.attend(0, q, k, v, HQ, HKV)
        assert torch.equal(o1, o2)
        fast.end_forward(c1)
        slow.end_forward(c2)
        assert np.array_equal(fast.pool.ref_count, slow.pool.ref_count)
        assert np.array_equal(fast.pool.tokens_used, slow.pool.tokens_used)

    step([5, 8, 1, 3], ids, expect_fast=False)       # prefill
    step([1, 1, 1, 1], ids, expect_fast=False)       # first decode: host plan
    for _ in range(13):                               # crosses page boundaries
        step([1, 1, 1, 1], ids, expect_fast=True)
    for m in (fast, slow):
        m.release_sequence("b")
    step([1, 1, 1], ["a", "c", "d"], expect_fast=False)  # batch changed
    step([1, 1, 1], ["a", "c", "d"], expect_fast=True)
    # a shared last page (refcount 2) must go through copy-on-write on the host
    for m in (fast, slow):
        m.pool.add_ref(int(m.seqs["c"].bt[m.seqs["c"].n_pages - 1]))
    step([1, 1, 1], ["a", "c", "d"], expect_fast=False)
    step([1, 1, 1], ["a", "c", "d"], expect_fast=True)
    # pages taken ahead by extend_sequence (their zeroing deferred): the host plans
    for m in (fast, slow):
        m.extend_sequence("a", 9)
    step([1, 1, 1], ["a", "c", "d"], expect_fast=False)
    for _ in range(10):
        step([1, 1, 1], ["a", "c", "d"])


def test_steady_decode_step_out_of_pages_matches_oracle():
    """A steady decode step that needs more pages than are free leaves the one-pass
    path untouched and fails in the general one, with the reference's error, at the
    same step as the oracle, both caches unchanged by the failed step."""
    g = torch.Generator().manual_seed(3)
    mgr, ref = make(ps=4, pages=12, prefix=False)
    ids = ["a", "b", "c"]
    for m in (mgr, ref):
        for s, n in zip(ids, [4, 7, 11]):
            m.allocate_sequence(s, num_tokens=n)
    forward_both(mgr, ref, ids, [4, 7, 11], [0, 0, 0], g)
    for step in range(40):
        errs = []
        for m in (mgr, ref):
            try:
                c = m.begin_forward(ids, [1, 1, 1])
            except RuntimeError as e:
                errs.append(str(e))
                continue
            m.end_forward(c) if m is ref else None
            if m is mgr:
                q = torch.randn(3, 1, HQ, D, generator=g)
                kv = torch.randn(3, 1, HKV, D, generator=g)
                c.attend(0, q, kv, kv, HQ, HKV)
                m.end_forward(c)
        if errs:
            assert len(errs) == 2 and errs[0] == errs[1] and errs[0].startswith("KV OOM"), errs
            break
        assert mgr.pool.num_free == ref.pool.num_free
    else:
        raise AssertionError("the pool never ran out")
    assert [mgr.seqs[s].num_tokens for s in ids] == [ref.seqs[s].num_tokens for s in ids]


@pytest.mark.parametrize("backend", ["paged", "contiguous"])
def test_attend_rope_equals_attend_on_rotated_inputs(backend):
    """attend_rope (rotation fused into the cache write) gives the same outputs and
    cache contents as the model's own sequence: positions from get_position_ids,
    eager rotation of q and k_new (models.py:96-103), then attend. Ragged prefill with
    input offsets, then decode steps (the device-planned ones included)."""
    g = torch.Generator().manual_seed(21)
    cos, sin = O.rope_tables(D, 512, 10000.0)
    cfg = dict(num_layers=L, num_kv_heads=HKV, num_qo_heads=HQ, head_dim=D, page_size=4, max_pages=64,
               dtype=torch.float16, device=None, backend=backend, max_batch_size=4, max_seq_len=128)
    if backend == "paged":
        a, b = (KC.PagedKVCache(KC.KVCacheConfig(**cfg), kernels=FK) for _ in range(2))
    else:
        a, b = (KC.ContiguousKVCache(KC.KVCacheConfig(**cfg), kernels=FK) for _ in range(2))
    ids = ["x", "y", "z"]
    for m in (a, b):
        for s, n in zip(ids, [6, 9, 3]):
            m.allocate_sequence(s, num_tokens=n)
    steps = [([6, 9, 3], [2, 0, 1])] + [([1, 1, 1], None)] * 6
    for ntok, offs in steps:
        offs = offs or [0] * len(ids)
        S = max(o + n for o, n in zip(offs, ntok))
        q = torch.randn(3, S, HQ, D, generator=g).half()
        k = torch.randn(3, S, HKV, D, generator=g).half()
        v = torch.randn(3, S, HKV, D, generator=g).half()
        ca, cb = a.begin_forward(ids, ntok, offs), b.begin_forward(ids, ntok, offs)
        for layer in range(L):
            oa = KC.attention_forward(q, k, v, layer, HQ, HKV, cos, sin, ca)
            pos = cb.get_position_ids(S)
            qr, kr = O.rope_forward_ref(q, k, cos, sin, pos)
            ob = cb.attend(layer, qr, kr, v, HQ, HKV)
            for bi in range(3):
                rows = slice(offs[bi], offs[bi] + ntok[bi])
                assert torch.equal(oa[bi, rows], ob[bi, rows])
        a.end_forward(ca)
        b.end_forward(cb)
        if backend == "paged":
            assert torch.equal(a.pool.k, b.pool.k) and torch.equal(a.pool.v, b.pool.v)
        else:
            assert torch.equal(a.k, b.k) and torch.equal(a.v, b.v)
    with pytest.raises(IndexError):
        short = O.rope_tables(D, 8, 10000.0)
        c = a.begin_forward(ids, [1, 1, 1])
        KC.attention_forward(q[:, :1], k[:, :1], v[:, :1], 0, HQ, HKV, short[0], short[1], c)


def test_decode_batch_with_shared_prefix_forms_groups():
    """A decode batch of requests admitted on one cached prompt: their first pages are
    the same pages, so the plan groups them (at most 16 / G rows per group, with the
    full pages they share below their last page) and the decode gets the groups; the
    steady steps planned on the device keep them. Outputs equal the oracle's."""
    g = torch.Generator().manual_seed(8)
    mgr, ref = make(ps=4, pages=160, prefix=True)
    prompt = list(range(1, 30))  # 7 full pages + 1 token
    for impl in (mgr, ref):
        impl.allocate_sequence("p", token_ids=prompt)
    forward_both(mgr, ref, ["p"], [len(prompt)], [0], g)
    for impl in (mgr, ref):
        impl.release_sequence("p")
    ids = [f"r{i}" for i in range(10)]
    for i, sid in enumerate(ids):
        toks = prompt[:28] + [100 + i] * (3 + i)
        for impl in (mgr, ref):
            assert impl.allocate_sequence(sid, token_ids=toks) == 28
    forward_both(mgr, ref, ids, [3 + i for i in range(10)], [0] * 10, g)
    seen = []
    for _ in range(6):
        FK.CALLS.clear()
        forward_both(mgr, ref, ids, [1] * 10, [0] * 10, g)
        launches = [grp for name, grp in FK.CALLS if name == "DecodeLaunch"]
        assert launches and launches[0] is not None
        seen.append(launches[0])
    grp = seen[0]
    M = 16 // (HQ // HKV)
    assert sorted(b for ms in grp.members for b in ms) == list(range(10))
    assert all(2 <= len(ms) <= M for ms in grp.members)
    assert grp.prefix_pages == [7] * grp.num_groups
    for ms in grp.members:  # the rows of a group share their first 7 pages
        tabs = [mgr.seqs[ids[b]].bt[:7].tolist() for b in ms]
        assert all(t == tabs[0] for t in tabs)
    assert all(s is grp for s in seen[1:])  # carried over by the device-planned steps


@pytest.mark.parametrize("scenario", ["prefill_then_decode", "cow_order", "radix_random", "positions",
                                      "csr", "attend_rope"])
def test_forward_plan_expanded_on_the_device_matches(scenario, monkeypatch):
    """The same scenarios with every multi-token forward's per-token plan expanded by
    the device planner (here its CPU stand-in) from the numpy path's host part (the
    native planner off): the oracle comparisons of each scenario still hold."""
    monkeypatch.setattr(KC.PagedCacheContext, "DEVICE_PLAN_TOKENS", 2)
    monkeypatch.setattr(KC.PagedKVCache, "NATIVE_PLAN", False)  # the numpy path's device plan
    FK.CALLS.clear()
    {"prefill_then_decode": test_prefill_then_decode_matches_oracle,
     "cow_order": test_copy_on_write_order_rule,
     "radix_random": test_radix_random_workload_matches_oracle,
     "positions": test_positions_shapes,
     "csr": test_csr_plan_closed_form,
     "attend_rope": lambda: test_attend_rope_equals_attend_on_rotated_inputs("paged")}[scenario]()
    if scenario in ("prefill_then_decode", "radix_random", "attend_rope"):  # these have multi-token forwards
        assert any(name == "forward_plan" for name, _ in FK.CALLS)


def _partial_sharing_scenario(impl, g):
    """The known-answer case of partial-page sharing (page size 4), on one cache:
    returns the values the test checks. A 10-token prompt (2 full pages + 2 tokens)
    is prefilled and released: the tree caches its 3 pages, the last one partial.
    Then B (the prompt + 2 tokens) matches all 10 tokens and shares the partial page;
    C and E diverge inside it and match the 2 full pages only; D (the prompt itself)
    matches it whole. B's first write lands in slot 2 of the shared page, which the
    tree, B and D hold: B copies it."""
    ps = 4
    prompt = list(range(1, 11))
    out = {}
    impl.allocate_sequence("A", token_ids=prompt)
    q = torch.randn(1, 10, HQ, D, generator=g)
    k = torch.randn(1, 10, HKV, D, generator=g)
    v = torch.randn(1, 10, HKV, D, generator=g)
    c = impl.begin_forward(["A"], [10])
    for layer in range(L):
        c.attend(layer, q, k, v, HQ, HKV)
    impl.end_forward(c)
    a_pages = list(impl.seqs["A"].block_table)
    impl.release_sequence("A")
    out["cached"] = impl.tree.cached_pages
    out["free_after_release"] = impl.pool.num_free
    out["plen"] = {s: impl.allocate_sequence(s, token_ids=t) for s, t in
                   (("B", prompt + [11, 12]), ("C", prompt[:9] + [99]), ("D", prompt), ("E", prompt[:9]))}
    out["B_shares_A_pages"] = list(impl.seqs["B"].block_table) == a_pages
    out["ref_partial"] = int(impl.pool.ref_count[a_pages[2]])
    c = impl.begin_forward(["B"], [2])
    kb = torch.randn(1, 2, HKV, D, generator=g)
    for layer in range(L):
        c.attend(layer, torch.randn(1, 2, HQ, D, generator=g), kb, kb, HQ, HKV)
    impl.end_forward(c)
    cow = c.cow_pairs if hasattr(c, "cow_pairs") else c.cow_events
    out["cow"] = [(int(s), int(d)) for s, d in cow]
    b3 = impl.seqs["B"].block_table[2]
    out["B_page3_is_copy"] = b3 != a_pages[2] and out["cow"] == [(a_pages[2], b3)]
    out["tokens_used"] = (int(impl.pool.tokens_used[a_pages[2]]), int(impl.pool.tokens_used[b3]))
    out["ref_after"] = int(impl.pool.ref_count[a_pages[2]])
    # B's K at positions 8, 9 are A's (copied), 10, 11 the new ones
    kk = impl.pool.k
    out["B_k"] = torch.stack([kk[0, b3, s] for s in range(4)]).float()
    out["A_k89"] = k[0, 8:10].float()
    out["new_k"] = kb[0].float()
    out["shared_untouched"] = torch.equal(kk[0, a_pages[2], :2].float(), k[0, 8:10].float())
    return out


def test_partial_page_sharing_known_answer():
    """Partial-page radix sharing, the same known answers from the oracle and the product
    (each checked on its own): cached pages, prefix lengths, refcounts, the single
    copy-on-write and the copied page's contents and tokens_used."""
    for impl in make(ps=4, pages=32, prefix=True, partial=True):
        out = _partial_sharing_scenario(impl, torch.Generator().manual_seed(12))
        assert out["cached"] == 3 and out["free_after_release"] == 31 - 3
        assert out["plen"] == {"B": 10, "C": 8, "D": 10, "E": 8}
        assert out["B_shares_A_pages"]
        assert out["ref_partial"] == 3  # the tree, B and D
        assert out["B_page3_is_copy"]
        assert out["tokens_used"] == (2, 4)  # the source keeps its 2 tokens; the copy has 4
        assert out["ref_after"] == 2  # the tree and D
        assert torch.equal(out["B_k"][:2], out["A_k89"]) and torch.equal(out["B_k"][2:], out["new_k"])
        assert out["shared_untouched"]
    # with the reference's rule (full pages only) the same prompts match whole pages only
    for impl in make(ps=4, pages=32, prefix=True, partial=False):
        out = _partial_sharing_scenario(impl, torch.Generator().manual_seed(12))
        assert out["cached"] == 2 and out["plen"] == {"B": 8, "C": 8, "D": 8, "E": 8}
        assert out["cow"] == []


@pytest.mark.parametrize("seed", range(6))
def test_partial_page_match_brute_force(seed):
    """match on released sequences (no eviction) against a tree-free rule: the full
    pages are the longest common prefix with a cached sequence, in whole pages of it;
    a partial page is the last page of a cached sequence whose tokens the prompt
    continues exactly and that ends inside the page after those full pages."""
    rnd = random.Random(seed)
    ps = rnd.choice([2, 3, 4])
    cfg = KC.KVCacheConfig(num_layers=1, num_kv_heads=1, num_qo_heads=1, head_dim=8, page_size=ps,
                           max_pages=400, dtype=torch.float32, device=None, enable_prefix_caching=True,
                           backend="paged", share_partial_pages=True)
    for impl in (KC.PagedKVCache(cfg, kernels=FK), O.PagedRef(1, 400, ps, 1, 8, share_partial_pages=True)):
        cached = []
        for i in range(12):
            toks = [rnd.randint(0, 1) for _ in range(rnd.randint(1, 4 * ps))]
            impl.allocate_sequence(f"s{i}", token_ids=toks)
            impl.seqs[f"s{i}"].num_tokens = len(toks)
            impl.release_sequence(f"s{i}")
            cached.append(toks)
        rnd2 = random.Random(seed + 100)
        for j in range(30):
            prompt = [rnd2.randint(0, 1) for _ in range(rnd2.randint(1, 5 * ps))]

            def lcp(a, b):
                n = 0
                while n < min(len(a), len(b)) and a[n] == b[n]:
                    n += 1
                return n
            f = max(min(lcp(prompt, s), len(s)) // ps for s in cached)
            r = max([len(s) - f * ps for s in cached
                     if len(s) % ps and len(s) // ps == f and lcp(prompt, s) >= len(s)] or [0])
            plen, pages = impl.tree.match(prompt)
            assert plen == f * ps + r, (impl, prompt)
            assert len(pages) == f + (1 if r else 0)


def test_pages_written_in_full_skip_the_owed_zeroing():
    """A multi-token forward zeroes the pages it owes zero-on-alloc (kv_cache.py:411)
    except those its own append writes in every slot: chunks of whole pages launch no
    zeroing, a chunk that ends inside a page zeroes that page. Every page of every
    block table, unwritten slots included, equals the oracle's bytes."""
    g = torch.Generator().manual_seed(21)
    mgr, ref = make(ps=4, pages=64, prefix=False)
    # pages written once and released, so the pages taken below hold old K/V
    for impl in (mgr, ref):
        impl.allocate_sequence("x")
    forward_both(mgr, ref, ["x"], [60], [0], g)
    for impl in (mgr, ref):
        impl.release_sequence("x")
    ids = ["a", "b"]
    for impl in (mgr, ref):
        for sid in ids:
            impl.allocate_sequence(sid)

    def zero_calls():
        return [n for name, n in FK.CALLS if name == "zero_pages"]

    FK.CALLS.clear()
    forward_both(mgr, ref, ids, [8, 12], [0, 0], g)  # whole pages only
    assert zero_calls() == []
    FK.CALLS.clear()
    forward_both(mgr, ref, ids, [6, 3], [0, 0], g)  # a: 8..13 ends inside a page; b: 12..14 too
    assert zero_calls() == [2]
    FK.CALLS.clear()
    forward_both(mgr, ref, ids, [2, 8], [0, 0], g)  # a fills its page; b: 15..22, a page in full
    assert zero_calls() == [1]  # and b's last page, slots 20..22 of 20..23
    check_state(mgr, ref, ids)
    for sid in ids:
        bt1, bt2 = mgr.seqs[sid].bt[:mgr.seqs[sid].n_pages].tolist(), ref.seqs[sid].block_table
        assert len(bt1) == len(bt2)
        for p1, p2 in zip(bt1, bt2):
            assert torch.equal(mgr.pool.k[:, p1], ref.pool.k[:, p2])
            assert torch.equal(mgr.pool.v[:, p1], ref.pool.v[:, p2])


def test_graph_context_refers_to_its_graph_weakly():
    """A DecodeGraph holds its step contexts and the contexts refer back to it weakly:
    a graph is freed by reference counting when its caller drops it, never later by
    the cyclic collector, which could run while another graph is being captured."""
    import gc
    import weakref

    class Holder:  # holds its contexts as DecodeGraph does
        seq_ids = ["a", "b"]
        rope_rows = None

    h = Holder()
    h.ctxs = [KC._GraphDecodeContext(h, None, None) for _ in range(2)]
    assert h.ctxs[0]._graph() is h
    wr = weakref.ref(h)
    was = gc.isenabled()
    gc.disable()
    try:
        del h
        assert wr() is None
    finally:
        if was:
            gc.enable()

